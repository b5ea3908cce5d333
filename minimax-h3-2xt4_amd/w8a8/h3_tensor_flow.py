"""FP16-fix tensor flow: residual divisor folding and the residual updates.

Mirrors the linear-path parts of patches/h3_tensor_flow.py: TensorFlowPolicy
(:16-37), StableNorm / stable_norms (:48-79), fold_linear (:82-103; the
divisor goes into the FP32 INT8 weight scales of the row projections),
prepare_tp (:114-127: projection folds, StableNorm, norm eps / c**2),
residual_add (:130-131), modulated_norm (:134-142) and gated_add
(:145-152), plus the DiT modulation segment -> row-label map of
patches/tilelang_dit_fusion.py:93-124.

For residual rows stored as y = x / c, an RMSNorm with eps / c**2 gives the
same normalized rows as the unscaled stream with eps: with c a power of two
every scaling step is exact in fp32, so the fold changes no bit.
"""
from dataclasses import dataclass

import torch
from torch import nn

from . import kernels


@dataclass(frozen=True)
class TensorFlowPolicy:
    mode: str = 'legacy'
    residual_exponent: int = 9
    vision_residual_exponent: int = 0
    video_residual_exponent: int = 0

    def __post_init__(self):
        if self.mode not in ('legacy', 'fp16', 'bf16_reference'):
            raise ValueError('Unknown H3 tensor flow')
        for value in (self.residual_exponent, self.vision_residual_exponent, self.video_residual_exponent):
            if type(value) is not int or not 0 <= value <= 12:
                raise ValueError('Residual exponent must be an integer in [0,12]')

    @property
    def enabled(self):
        return self.mode != 'legacy'

    @property
    def dtype(self):
        return torch.bfloat16 if self.mode == 'bf16_reference' else torch.float16

    @property
    def divisor(self):
        return float(2 ** self.residual_exponent)


class StableNorm(nn.Module):
    """FP32 statistics, gain and epsilon, then the activation storage cast
    (patches/h3_tensor_flow.py:48-69). ``eps`` is the wrapped norm's epsilon
    divided by divisor**2. RMSNorm only: the LayerNorm variant belongs to
    the vision/VAE paths this build leaves out.

    Calling it on 16-bit rows on the GPU runs the library's RMSNorm kernel
    (fixed-order fp32 sum of squares, IEEE sqrt and division); FP32 rows run
    torch's F.rms_norm in fp32, the reference's own expression. The DiT
    sublayers read ``weight`` and ``eps`` from it and fuse the norm into the
    next projection's quantization.
    """

    def __init__(self, norm, divisor=1.):
        super().__init__()
        if 'LayerNorm' in type(norm).__name__ or getattr(norm, 'layer_norm', False):
            raise ValueError('StableNorm here wraps RMSNorm modules only')
        self.weight = norm.weight
        self.normalized_shape = tuple(norm.normalized_shape)
        eps = norm.eps if norm.eps is not None else torch.finfo(torch.float32).eps
        self.eps = float(eps) / (divisor * divisor)
        self.layer_norm = False

    def forward(self, x):
        if x.is_cuda and x.dtype in (torch.float16, torch.bfloat16) and len(self.normalized_shape) == 1:
            weight = self.weight.detach().to(device=x.device, dtype=torch.float32) if self.weight is not None \
                else None
            flat = x.reshape(-1, x.shape[-1])
            y = kernels.norm_quantize(flat, weight, eps=self.eps, quantize=False)['y']
            return y.reshape(x.shape)
        weight = self.weight.to(device=x.device, dtype=torch.float32) if self.weight is not None else None
        return torch.nn.functional.rms_norm(x.float(), self.normalized_shape, weight, self.eps).to(x.dtype)


def stable_norms(module):
    """Replace every norm child (anything with normalized_shape and eps) by
    a StableNorm, recursively (patches/h3_tensor_flow.py:72-79)."""
    for name, child in list(module.named_children()):
        if isinstance(child, StableNorm):
            continue
        if hasattr(child, 'normalized_shape') and hasattr(child, 'eps'):
            setattr(module, name, StableNorm(child))
        else:
            stable_norms(child)


def fold_linear(module, divisor):
    """Divide the FP32 INT8 weight scale (and any bias) by the divisor once.

    The divisor is a power of two, so the fold is exact for normal values.
    """
    base = getattr(module, 'base', module)
    if not hasattr(base, 'weight_scale'):
        raise ValueError('Residual folding requires an INT8 projection with FP32 weight scales')
    base.weight_scale = nn.Parameter(base.weight_scale.detach().float() / divisor, requires_grad=False)
    bias = getattr(base, 'bias', None)
    if bias is not None:
        base.bias = nn.Parameter(bias.detach() / divisor, requires_grad=False)


def prepare_tp(block, kind, policy):
    """Prepare a block for the scaled residual flow (patches/h3_tensor_flow.py:114-127).

    Folds the divisor c into the row projections (out_proj/fc2 for DiT,
    o_proj/down_proj for TE), installs StableNorm in place of every norm,
    and divides the eps of the residual-stream norms (norm1/norm2 for DiT,
    input_layernorm/post_attention_layernorm for TE) by c**2. A sub-block
    that holds only some of these (e.g. an FFN sublayer, whose norm the
    caller passes in) gets the folds for what it holds.
    """
    if not policy.enabled:
        return block
    if hasattr(block, 'tensor_flow'):
        raise ValueError('Tensor flow already prepared')
    block.tensor_flow = policy
    c = policy.divisor
    for name in (('o_proj', 'down_proj') if kind == 'te' else ('out_proj', 'fc2')):
        module = getattr(block, name, None)
        if module is not None:
            fold_linear(module, c)
    stable_norms(block)
    for name in (('input_layernorm', 'post_attention_layernorm') if kind == 'te' else ('norm1', 'norm2')):
        norm = getattr(block, name, None)
        if norm is not None:
            norm.eps /= c * c
    return block


def residual_add(x, branch):
    """x = cast(f32(x) + f32(branch)) to x's dtype."""
    return (x.float() + branch.float()).to(x.dtype)


def segment_key(rows, segments, modulation_rows=9):
    """Canonical segments when they tile [0, rows) exactly with valid table
    rows, else None (patches/tilelang_dit_fusion.py:93-100)."""
    key = tuple(tuple(seg) for seg in segments)
    cursor = 0
    for a, b, row in sorted(key):
        if (any(type(v) is not int for v in (a, b, row)) or a != cursor
                or not a < b <= rows or not 0 <= row < modulation_rows):
            return None
        cursor = b
    return key if cursor == rows else None


def labels_for(rows, segments, modulation_rows=9, device=None):
    """int32 [rows] gate-table row of every row, or None when the segments do
    not tile the rows (patches/tilelang_dit_fusion.py:106-124)."""
    key = segment_key(rows, segments, modulation_rows)
    if key is None:
        return None
    labels = torch.empty(rows, dtype=torch.int32)
    for a, b, row in key:
        labels[a:b] = row
    return labels.to(device) if device is not None else labels


def gated_add(x, gate, branch, segments):
    """Eager DiT gated residual update (:145-152): per segment,
    x[a:b] = cast(f32(x) + f32(branch) * gate[row]) with torch.addcmul.

    The fused route (the GEMM epilogue with gate=/gate_labels=) computes the
    same update with one fp32 FMA rounding, as the reference's fused
    row_gate_kernel does; torch.addcmul's own rounding is not pinned.
    """
    for a, b, row in segments:
        x[a:b].copy_(torch.addcmul(x[a:b].float(), branch[a:b].float(), gate[row].float()).to(x.dtype))
    return x


def _norm_args(norm, x, shift, scale, segments):
    if x.ndim != 2:
        raise ValueError('modulated_norm expects [tokens, hidden] rows')
    if tuple(norm.normalized_shape) != (x.shape[1],) or getattr(norm, 'layer_norm', False):
        raise ValueError('an RMSNorm over the hidden dimension is required')
    weight = getattr(norm, 'weight', None)
    if weight is not None:
        weight = weight.detach().to(device=x.device, dtype=torch.float32)
    eps = norm.eps if norm.eps is not None else torch.finfo(torch.float32).eps
    labels = None
    if shift is not None:
        labels = labels_for(x.shape[0], segments, shift.shape[0], device=x.device)
        if labels is None:
            raise ValueError('segments must tile the rows with valid modulation-table rows')
        shift = shift.to(torch.float32)
        scale = scale.to(torch.float32)
    return weight, eps, labels, shift, scale


def modulated_norm(norm, x, shift, scale, segments, *, fused=False):
    """DiT modulated RMSNorm (patches/h3_tensor_flow.py:134-142, fused route
    patches/tilelang_dit_fusion.py:10-36,127-135) on the libw8a8 kernel:

    y = cast((((x * inv) * w) * (1 + scale[row])) + shift[row]) per segment
    row, inv = 1 / sqrt(mean(x*x) + eps), in fp32. ``fused`` is accepted for
    API compatibility; both routes run the one kernel (the sum of squares in
    its fixed order, IEEE sqrt and division in place of rsqrtf). shift and
    scale are the [R, hidden] modulation tables; None for a plain RMSNorm.
    """
    weight, eps, labels, shift, scale = _norm_args(norm, x, shift, scale, segments)
    return kernels.norm_quantize(x, weight, shift, scale, labels, eps=eps, quantize=False)['y']


def modulated_norm_quantize(norm, x, shift, scale, segments, *, convrot=True, convrot_groupsize=256,
                            want_normalized=False):
    """modulated_norm fused with the column path's activation preparation
    (ConvRot256 rounded to x's dtype, then per-row INT8): returns
    (codes int8 [M, hidden], row_scale fp32 [M, 1]) and, with
    want_normalized, the normalized rows as a third item. The codes equal
    those of quantizing modulated_norm's output (patches/dit_column_linear.py:13-21).
    """
    if convrot and convrot_groupsize != 256:
        raise ValueError('only the regular-H4 ConvRot256 group size is supported')
    weight, eps, labels, shift, scale = _norm_args(norm, x, shift, scale, segments)
    r = kernels.norm_quantize(x, weight, shift, scale, labels, eps=eps, convrot=bool(convrot),
                              want_normalized=want_normalized)
    if want_normalized:
        return r['q'], r['scale'], r['y']
    return r['q'], r['scale']
