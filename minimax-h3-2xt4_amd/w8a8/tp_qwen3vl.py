"""Text-encoder INT8 projections (the reference's tp_qwen3vl API) on one GPU.

ColumnParallelLinearINT8 / RowParallelLinearINT8 keep the names and
attributes of patches/tp_qwen3vl.py:25-115 (weight int8 [N, K],
weight_scale fp32 [N, 1], convrot, convrot_groupsize, rank, world_size,
in/out features); the TE column split is a contiguous row range (no packed
components). RowParallelLinearINT8.forward_parts is the TE down projection
from separate gate/up halves (:113-115), project_columns shares one
activation quantization among the column projections that read the same
rows (:121-134), and TEFeedForwardINT8 is the MLP half of
TPTransformerBlockINT8.forward (:259-281) in the scaled FP16 flow.
"""
import torch
from torch import nn

from . import kernels, parallel_int8
from .dit_column_linear import column_linear, column_linear_quantized
from .h3_operator_policy import H3OperatorPolicy, row_linear as dispatch_row, row_linear_parts


class ColumnParallelLinearINT8(nn.Module):
    """Output-feature split INT8 projection of the text encoder (patches/tp_qwen3vl.py:25-67)."""

    def __init__(self, in_features, out_features, rank=0, world_size=1, convrot=True, convrot_groupsize=256,
                 device=None):
        super().__init__()
        if out_features % world_size:
            raise ValueError('out_features must divide across ranks')
        self.in_features = in_features
        self.out_features_per_rank = out_features // world_size
        self.rank = rank
        self.world_size = world_size
        self.convrot = convrot
        self.convrot_groupsize = convrot_groupsize
        self.device = torch.device(device) if device is not None else torch.device('cuda', 0)
        self.weight = nn.Parameter(torch.empty(self.out_features_per_rank, in_features, dtype=torch.int8,
                                               device=self.device), requires_grad=False)
        self.weight_scale = nn.Parameter(torch.empty(self.out_features_per_rank, 1, dtype=torch.float32,
                                                     device=self.device), requires_grad=False)

    def load_shard_from_full(self, full_weight, full_scale):
        start = self.rank * self.out_features_per_rank
        end = start + self.out_features_per_rank
        self.weight.data.copy_(full_weight[start:end, :])
        self.weight_scale.data.copy_(full_scale[start:end, :])

    def forward(self, x, *, prepared=None, out=None):
        """Kitchen int8_linear (rotate, quantize, GEMM, column dequant) on
        the library's kernels: column_linear with x's dtype as output.
        ``prepared`` (codes, row_scale) skips the quantization; ``out`` (a
        [rows, N] view, e.g. columns of a packed buffer) receives the result."""
        if self.convrot and self.convrot_groupsize != 256:
            raise ValueError('only the regular-H4 ConvRot256 group size is supported')
        flat = x.reshape(-1, self.in_features)
        if prepared is None and out is None:
            y = column_linear(flat, self.weight, self.weight_scale, convrot=self.convrot,
                              convrot_groupsize=self.convrot_groupsize, out_dtype=x.dtype)
        else:
            if prepared is None:
                prepared = kernels.quantize_rows(flat, convrot=bool(self.convrot), round_rotated=True)
            y = _column_into(prepared[0], prepared[1], self.weight, self.weight_scale, x.dtype, out)
        return y.view(*x.shape[:-1], self.out_features_per_rank)


def _column_into(codes, row_scale, weight, weight_scale, out_dtype, out):
    if out is None:
        return column_linear_quantized(codes, row_scale, weight, weight_scale, out_dtype=out_dtype)
    scale = weight_scale.to(device=codes.device, dtype=torch.float32).reshape(-1)
    return kernels.gemm(codes, weight, epilogue=kernels.EPI_COLUMN, row_scale=row_scale, col_scale=scale,
                        out_dtype=out_dtype, out=out)


class RowParallelLinearINT8(nn.Module):
    """Input-feature split INT8 projection of the text encoder (patches/tp_qwen3vl.py:70-115)."""

    def __init__(self, in_features, out_features, rank=0, world_size=1, convrot=True, convrot_groupsize=256,
                 device=None):
        super().__init__()
        if in_features % world_size:
            raise ValueError('in_features must divide across ranks')
        self.in_features_per_rank = in_features // world_size
        self.out_features = out_features
        self.rank = rank
        self.world_size = world_size
        self.convrot = convrot
        self.convrot_groupsize = convrot_groupsize
        self.device = torch.device(device) if device is not None else torch.device('cuda', 0)
        self.weight = nn.Parameter(torch.empty(out_features, self.in_features_per_rank, dtype=torch.int8,
                                               device=self.device), requires_grad=False)
        self.weight_scale = nn.Parameter(torch.empty(out_features, 1, dtype=torch.float32, device=self.device),
                                         requires_grad=False)

    def load_shard_from_full(self, full_weight, full_scale):
        start = self.rank * self.in_features_per_rank
        end = start + self.in_features_per_rank
        self.weight.data.copy_(full_weight[:, start:end])
        self.weight_scale.data.copy_(full_scale)

    def _single_rank(self):
        if self.world_size != 1:
            raise ValueError('a TE row shard needs the SUM exchange; this build runs whole TE projections')

    def forward(self, x, reduce_sum=True):
        """Row projection (patches/tp_qwen3vl.py:103-110): dispatch by the
        operator policy, result in x's dtype."""
        if not reduce_sum and self.world_size > 1:
            raise ValueError('Quantization-preserving row projection requires reduction')
        self._single_rank()
        return dispatch_row(self, x, parallel_int8.row_linear, None).to(x.dtype)

    def forward_parts(self, gate, up, *, residual=None):
        """Down projection of separate gate/up halves (patches/tp_qwen3vl.py:112-115
        -> h3_operator_policy.row_linear_parts), result in gate's dtype.

        With ``residual`` (FP16, the scaled residual stream) on the fused
        route the TE update fp16(f32(residual) + f32(fp16(branch)))
        (h3_tensor_flow.residual_add) runs in the GEMM epilogue and the
        updated residual is returned; it equals residual_add(residual,
        forward_parts(gate, up)) bit for bit.
        """
        self._single_rank()
        if residual is None:
            return row_linear_parts(self, gate, up, parallel_int8.row_linear, None).to(gate.dtype)
        policy = getattr(self, 'operator_policy', None)
        fused = (policy is not None and policy.row_linear_backend != 'native'
                 and policy.fc2_quantizer in ('fused_stored', 'fused_recompute'))
        if not fused or gate.dtype != torch.float16 or residual.dtype != torch.float16:
            from .h3_tensor_flow import residual_add
            return residual_add(residual, self.forward_parts(gate, up))
        if gate.shape != up.shape or gate.dtype != up.dtype or gate.device != up.device:
            raise ValueError('Matching gate/up required')
        from .h3_operator_policy import adjacent_cat, row_linear
        return row_linear(self, adjacent_cat(gate, up), parallel_int8.row_linear, None, 'swiglu',
                          residual=residual)


def project_columns(x, *modules):
    """Column projections of the same rows (patches/tp_qwen3vl.py:121-134).

    When every module is a plain ColumnParallelLinearINT8 (no hooks, no
    forward override) with the same ConvRot settings, x is rotated and
    quantized once and each projection is one GEMM, its output written into
    its own columns of one packed [rows, sum N] buffer (so gate and up of
    the MLP sit side by side). The reference takes this route only at the
    TE hidden size 5120; here it is taken at any width, since sharing the
    quantization changes no bit of any output. Otherwise each module runs
    on its own.
    """
    plain = (len(modules) > 0 and all(
        type(m) is ColumnParallelLinearINT8 and 'forward' not in m.__dict__ and not m._forward_hooks
        and not m._forward_pre_hooks and (m.convrot, m.convrot_groupsize) == (modules[0].convrot,
                                                                            modules[0].convrot_groupsize)
        and m.in_features == x.shape[-1] for m in modules)
        and not nn.modules.module._global_forward_hooks and not nn.modules.module._global_forward_pre_hooks)
    if not plain:
        return tuple(m(x) for m in modules)
    m0 = modules[0]
    if m0.convrot and m0.convrot_groupsize != 256:
        raise ValueError('only the regular-H4 ConvRot256 group size is supported')
    flat = x.reshape(-1, x.shape[-1])
    codes, row_scale = kernels.quantize_rows(flat, convrot=bool(m0.convrot), round_rotated=True)
    widths = [m.out_features_per_rank for m in modules]
    packed = torch.empty((flat.shape[0], sum(widths)), dtype=x.dtype, device=x.device)
    outs, start = [], 0
    for m, w in zip(modules, widths):
        view = packed[:, start:start + w]
        m(x, prepared=(codes, row_scale), out=view)
        outs.append(view.view(*x.shape[:-1], w))
        start += w
    return tuple(outs)


class TEFeedForwardINT8(nn.Module):
    """The MLP half of the text-encoder block (patches/tp_qwen3vl.py:259-281)
    in the scaled FP16 flow: x <- x + down(silu(gate(n)) * up(n)) with
    n = rms_norm(x, post_attention_layernorm).

    The RMSNorm is fused into the shared gate/up activation quantization
    (its normalized rows never reach HBM; the codes equal those of
    quantizing the normalized rows), gate and up land side by side in one
    buffer, the down projection takes them through the fused FP32
    SwiGLU/ConvRot256 prologue, and the residual add runs in its epilogue.
    Run prepare_tp(ffn, 'te', policy) first (down_proj scale / divisor,
    StableNorm, eps / divisor**2).
    """

    def __init__(self, hidden, intermediate, *, eps=1e-6, device=None, policy=None):
        super().__init__()
        self.gate_proj = ColumnParallelLinearINT8(hidden, intermediate, device=device)
        dev = self.gate_proj.device
        self.up_proj = ColumnParallelLinearINT8(hidden, intermediate, device=dev)
        self.down_proj = RowParallelLinearINT8(intermediate, hidden, device=dev)
        self.post_attention_layernorm = nn.RMSNorm(hidden, eps=eps, device=dev, dtype=torch.float16)
        self.requires_grad_(False)
        policy = policy or H3OperatorPolicy()
        self.operator_policy = policy
        for m in (self.gate_proj, self.up_proj, self.down_proj):
            m.operator_policy = policy

    def forward(self, x):
        flow = getattr(self, 'tensor_flow', None)
        if flow is None:
            raise ValueError('the INT8 TE MLP runs the scaled tensor flow: prepare_tp(ffn, "te", policy) first')
        if x.dtype != flow.dtype:
            raise ValueError('TE residual dtype does not match tensor flow')
        norm = self.post_attention_layernorm
        flat = x.reshape(-1, x.shape[-1])
        weight = norm.weight.detach().to(device=x.device, dtype=torch.float32) if norm.weight is not None else None
        r = kernels.norm_quantize(flat, weight, eps=norm.eps, convrot=bool(self.gate_proj.convrot))
        gate, up = project_columns_prepared(flat, (r['q'], r['scale']), self.gate_proj, self.up_proj)
        out = self.down_proj.forward_parts(gate, up, residual=flat)
        return out.view(x.shape)


def project_columns_prepared(x, prepared, *modules):
    """project_columns for rows already rotated and quantized (codes,
    row_scale): each module's GEMM writes its columns of one packed buffer."""
    flat = x.reshape(-1, x.shape[-1])
    widths = [m.out_features_per_rank for m in modules]
    packed = torch.empty((flat.shape[0], sum(widths)), dtype=x.dtype, device=x.device)
    outs, start = [], 0
    for m, w in zip(modules, widths):
        view = packed[:, start:start + w]
        m(x, prepared=prepared, out=view)
        outs.append(view.view(*x.shape[:-1], w))
        start += w
    return tuple(outs)
