"""Typed wrappers of the libw8a8 entry points over torch device tensors.

Outputs are allocated here with torch (the library never allocates) and the
work is queued on the current stream of the tensors' device. Every wrapper
checks device, dtype, shape and layout first and raises ValueError on a
contract violation; a failing library call raises W8A8Error.
"""
import ctypes

import torch

from . import _abi
from ._abi import EPI_COLUMN, EPI_INT32, EPI_ROW  # noqa: F401

_OUT_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _device(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError('libw8a8 operates on HIP device tensors only (no CPU fallback)')
    dev = tensors[0].device
    for t in tensors:
        if t is not None and t.device != dev:
            raise ValueError('all tensors must be on the same device')
    return dev


def _rows_2d(x):
    """[rows, cols] view with unit column stride (row stride may exceed cols)."""
    if x.ndim != 2:
        x = x.reshape(-1, x.shape[-1])
    if x.stride(-1) != 1:
        x = x.contiguous()
    return x


def _scale_vec(s, n, name):
    s = s.to(dtype=torch.float32).reshape(-1)
    if not s.is_contiguous():
        s = s.contiguous()
    if s.numel() not in (1, n):
        raise ValueError(f'{name} must be scalar or have {n} entries')
    return s, (0 if s.numel() == 1 else 1)


def quantize_rows(x, *, convrot=False, round_rotated=True, row_max=None, out=None, scale_out=None, signs=None):
    """Per-row absmax INT8 quantization of x [M, K] -> (q int8 [M,K], scale fp32 [M,1]).

    convrot=True rotates each 256-column group first (regular-H4 ConvRot256);
    round_rotated rounds the rotated values to x's dtype before the absmax.
    row_max [M] (or [M,1]) fp32 replaces the row's own absmax. signs: the
    sign words of a seeded ConvRot (convrot.sign_words), with convrot.
    """
    x = _rows_2d(x)
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError('x must be float16, bfloat16 or float32')
    rows, cols = x.shape
    if convrot and cols % 256:
        raise ValueError('ConvRot group size must divide input features')
    if cols % 16:
        raise ValueError('input features must be a multiple of 16')
    if out is not None:
        if (out.dtype != torch.int8 or out.ndim != 2 or tuple(out.shape) != (rows, cols) or out.stride(1) != 1
                or out.stride(0) < cols or out.stride(0) % 16 or out.data_ptr() % 16):
            raise ValueError(f'out must be int8 [{rows}, {cols}] with unit column stride and 16-byte aligned rows')
    if scale_out is not None:
        if (scale_out.dtype != torch.float32 or tuple(scale_out.shape) not in ((rows, 1), (rows,))
                or (rows > 1 and scale_out.stride(0) != 1)):
            raise ValueError(f'scale_out must be contiguous float32 [{rows}, 1]')
    _device(x, row_max, out, scale_out)
    q = out if out is not None else torch.empty((rows, cols), dtype=torch.int8, device=x.device)
    scale = scale_out if scale_out is not None else torch.empty((rows, 1), dtype=torch.float32, device=x.device)
    if row_max is not None:
        row_max = row_max.to(torch.float32).reshape(-1).contiguous()
        if row_max.numel() != rows:
            raise ValueError('row_max must have one entry per row')
    if signs is not None and not convrot:
        raise ValueError('signs apply to the ConvRot256 rotation (convrot=True)')
    signs = _sign_words(signs, cols, x.device)
    if rows == 0:
        return q, scale
    args = _abi.QuantArgs(x_dtype=_abi.DTYPE_CODE[x.dtype], x=x.data_ptr(), ldx=x.stride(0), rows=rows, cols=cols,
                          convrot=256 if convrot else 0, round_rotated=1 if round_rotated else 0,
                          row_max=_abi.ptr(row_max), q=q.data_ptr(), ldq=q.stride(0), scale=scale.data_ptr(),
                          stream=_abi.stream_of(x), convrot_signs=_abi.ptr(signs))
    _abi.call('w8a8_quantize_rows', args)
    return q, scale


def row_absmax(x, *, convrot=False, round_rotated=True, signs=None):
    """Maximum phase of quantize_rows: fp32 [M, 1] row absmax of x [M, K]
    (after ConvRot256 when convrot), the value a tensor-parallel owner of a
    K slice contributes to the MAX exchange before quantizing with the
    global maximum (quantize_rows(row_max=...)). No codes are written.
    """
    x = _rows_2d(x)
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError('x must be float16, bfloat16 or float32')
    rows, cols = x.shape
    if (convrot and cols % 256) or cols % 16:
        raise ValueError('input features must be a multiple of 16 (256 with ConvRot256)')
    _device(x)
    if signs is not None and not convrot:
        raise ValueError('signs apply to the ConvRot256 rotation (convrot=True)')
    signs = _sign_words(signs, cols, x.device)
    res = torch.empty((rows, 1), dtype=torch.float32, device=x.device)
    if rows == 0:
        return res
    if cols == 0:
        return res.zero_()
    args = _abi.QuantArgs(x_dtype=_abi.DTYPE_CODE[x.dtype], x=x.data_ptr(), ldx=x.stride(0), rows=rows, cols=cols,
                          convrot=256 if convrot else 0, round_rotated=1 if round_rotated else 0,
                          row_max=None, q=None, ldq=0, scale=None, stream=_abi.stream_of(x),
                          row_max_out=res.data_ptr(), convrot_signs=_abi.ptr(signs))
    _abi.call('w8a8_quantize_rows', args)
    return res


def _sign_words(signs, cols, device):
    """Check a ConvRot sign-word tensor (convrot.sign_words): int32 [cols],
    contiguous and 16-byte aligned on device; None stays None."""
    if signs is None:
        return None
    if signs.dtype != torch.int32 or signs.numel() != cols or not signs.is_contiguous() or signs.data_ptr() % 16:
        raise ValueError(f'signs must be the int32 sign words of convrot.sign_words ({cols} entries, contiguous)')
    if signs.device != device:
        raise ValueError('all tensors must be on the same device')
    return signs


def _table(t, name, cols):
    if t.dtype != torch.float32 or t.ndim != 2 or t.shape[1] != cols:
        raise ValueError(f'{name} must be a float32 [rows, {cols}] table')
    if t.stride(1) != 1 or t.stride(0) % 4 or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def norm_quantize(x, weight=None, shift=None, scale=None, labels=None, *, eps, quantize=True, convrot=True,
                  round_rotated=True, want_normalized=False, signs=None):
    """Modulated RMSNorm of x [M, K] (F16/BF16), optionally fused with
    ConvRot256 and per-row INT8 quantization.

    y = x_dtype(((((x * inv) * weight) * (1 + scale[label])) + shift[label]))
    with inv = 1 / sqrt(sum(x*x) * fp32(1/K) + eps); weight [K] fp32 (None:
    no gain); shift/scale fp32 [R, K] AdaLN tables with labels int32 [M]
    (each row's table row), or None for a plain RMSNorm.
    Returns a dict with 'q' [M,K] int8 and 'scale' [M,1] fp32 when quantize,
    and 'y' [M,K] (x's dtype) when want_normalized or not quantize. signs:
    the sign words of a seeded ConvRot (convrot.sign_words), with quantize
    and convrot.
    """
    x = _rows_2d(x)
    _device(x, weight, shift, scale, labels)
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError('x must be float16 or bfloat16')
    rows, cols = x.shape
    if cols % 16 or (quantize and convrot and cols % 256):
        raise ValueError('input features must be a multiple of 16 (256 with ConvRot256)')
    if x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    if weight is not None:
        weight = weight.reshape(-1)
        if weight.dtype != torch.float32 or weight.numel() != cols:
            raise ValueError(f'weight must be float32 with {cols} entries')
        weight = weight.contiguous()
        if weight.data_ptr() % 16:
            weight = weight.clone()
    if (shift is None) != (scale is None):
        raise ValueError('shift and scale go together')
    if shift is not None:
        shift = _table(shift, 'shift', cols)
        scale = _table(scale, 'scale', cols)
        if scale.shape[0] != shift.shape[0] or scale.stride(0) != shift.stride(0):
            scale = scale.contiguous()
            shift = shift.contiguous()
            if scale.shape[0] != shift.shape[0]:
                raise ValueError('shift and scale tables must have the same rows')
        if labels is None or labels.dtype != torch.int32 or labels.numel() != rows:
            raise ValueError('modulation tables need int32 labels, one per row')
        labels = labels.reshape(-1).contiguous()
    if signs is not None and not (quantize and convrot):
        raise ValueError('signs apply to the ConvRot256 rotation of the quantized output')
    signs = _sign_words(signs, cols, x.device)
    out = {}
    want_y = want_normalized or not quantize
    y = torch.empty((rows, cols), dtype=x.dtype, device=x.device) if want_y else None
    q = torch.empty((rows, cols), dtype=torch.int8, device=x.device) if quantize else None
    qs = torch.empty((rows, 1), dtype=torch.float32, device=x.device) if quantize else None
    if quantize:
        out['q'], out['scale'] = q, qs
    if want_y:
        out['y'] = y
    if rows == 0:
        return out
    args = _abi.NormArgs(x_dtype=_abi.DTYPE_CODE[x.dtype], x=x.data_ptr(), ldx=x.stride(0), rows=rows, cols=cols,
                         weight=_abi.ptr(weight), mod_shift=_abi.ptr(shift), mod_scale=_abi.ptr(scale),
                         ld_mod=shift.stride(0) if shift is not None else 0,
                         mod_rows=shift.shape[0] if shift is not None else 0, eps=float(eps),
                         labels=_abi.ptr(labels), y=_abi.ptr(y), ldy=cols if y is not None else 0,
                         convrot=256 if convrot else 0, round_rotated=1 if round_rotated else 0,
                         q=_abi.ptr(q), ldq=cols if q is not None else 0, q_scale=_abi.ptr(qs),
                         stream=_abi.stream_of(x), convrot_signs=_abi.ptr(signs))
    _abi.call('w8a8_norm_quantize', args)
    return out


def rms_rope(packed, freqs, q_gain, k_gain, *, heads, rot_dim, eps, dim=128, out_dtype=torch.float16):
    """Per-head FP32 RMS norm + split-half RoPE of packed Q and K.

    packed: [rows, >= 2*heads*dim] fp16/fp32 (Q heads, then K heads; V may
    follow); freqs: [rows, rot_dim/2, 2, 2] fp16/fp32 rotation matrices;
    q_gain, k_gain: [dim]. Returns (q, k), each [rows, heads, dim] in out_dtype.
    """
    packed = _rows_2d(packed)
    _device(packed, freqs, q_gain, k_gain)
    if packed.dtype not in (torch.float16, torch.float32):
        raise ValueError('packed QKV must be float16 or float32')
    if freqs.dtype not in (torch.float16, torch.float32):
        raise ValueError('frequencies must be float16 or float32')
    if out_dtype not in (torch.float16, torch.float32):
        raise ValueError('output must be float16 or float32')
    rows = packed.shape[0]
    if dim != 128 or packed.shape[1] < 2 * heads * dim:
        raise ValueError('full 128-wide heads with Q and K in the packed row required')
    if not (0 < rot_dim <= dim and rot_dim % 2 == 0):
        raise ValueError('even rotary prefix required')
    def aligned(t):
        t = t.contiguous()
        return t if t.data_ptr() % 16 == 0 else t.clone()
    freqs = aligned(freqs.reshape(rows, rot_dim // 2, 2, 2))
    if packed.stride(0) * packed.element_size() % 16 or packed.data_ptr() % 16:
        packed = packed[:, :2 * heads * dim].contiguous()   # Q and K only: 16-byte rows
    gq = aligned(q_gain.to(torch.float32).reshape(-1))
    gk = aligned(k_gain.to(torch.float32).reshape(-1))
    if gq.numel() != dim or gk.numel() != dim:
        raise ValueError(f'gains must have {dim} entries')
    q = torch.empty((rows, heads, dim), dtype=out_dtype, device=packed.device)
    k = torch.empty((rows, heads, dim), dtype=out_dtype, device=packed.device)
    if rows == 0:
        return q, k
    args = _abi.RmsRopeArgs(in_dtype=_abi.DTYPE_CODE[packed.dtype], packed=packed.data_ptr(), ldp=packed.stride(0),
                            rows=rows, heads=heads, dim=dim, rot_dim=rot_dim,
                            freq_dtype=_abi.DTYPE_CODE[freqs.dtype], freqs=freqs.data_ptr(), q_gain=gq.data_ptr(),
                            k_gain=gk.data_ptr(), eps=float(eps), out_dtype=_abi.DTYPE_CODE[out_dtype],
                            q_out=q.data_ptr(), k_out=k.data_ptr(), stream=_abi.stream_of(packed))
    _abi.call('w8a8_rms_rope', args)
    return q, k


def swiglu_quantize(x, *, row_max=None, quantize=True, want_row_max=False, want_group_max=False, signs=None):
    """Fused FP32 SwiGLU -> ConvRot256 -> row absmax -> INT8 of x [M, 2W].

    Returns a dict with 'q' [M,W] int8 and 'scale' [M,1] fp32 (when
    quantize), 'row_max' [M,1] and 'group_max' [M,W/256] when requested.
    row_max (input) is an external absmax for the quantization. signs: the
    sign words of a seeded ConvRot (convrot.sign_words) of width W.
    """
    x = _rows_2d(x)
    _device(x, row_max)
    if x.dtype not in (torch.float16, torch.float32):
        raise ValueError('x must be float16 or float32')
    rows, two_w = x.shape
    width = two_w // 2
    if two_w != 2 * width or width % 256 or width == 0:
        raise ValueError('[M, 2W] input with W a positive multiple of 256 required')
    if not (quantize or want_row_max or want_group_max):
        raise ValueError('no output requested')
    dev = x.device
    res = {}
    if quantize:
        res['q'] = torch.empty((rows, width), dtype=torch.int8, device=dev)
        res['scale'] = torch.empty((rows, 1), dtype=torch.float32, device=dev)
    if want_row_max:
        res['row_max'] = torch.empty((rows, 1), dtype=torch.float32, device=dev)
    if want_group_max:
        res['group_max'] = torch.empty((rows, width // 256), dtype=torch.float32, device=dev)
    if row_max is not None:
        row_max = row_max.to(torch.float32).reshape(-1).contiguous()
        if row_max.numel() != rows:
            raise ValueError('row_max must have one entry per row')
    signs = _sign_words(signs, width, dev)
    if rows == 0:
        return res
    args = _abi.SwigluArgs(x_dtype=_abi.DTYPE_CODE[x.dtype], x=x.data_ptr(), ldx=x.stride(0), rows=rows,
                           width=width, row_max=_abi.ptr(row_max), row_max_out=_abi.ptr(res.get('row_max')),
                           group_max=_abi.ptr(res.get('group_max')), q=_abi.ptr(res.get('q')),
                           ldq=width, scale=_abi.ptr(res.get('scale')), stream=_abi.stream_of(x),
                           convrot_signs=_abi.ptr(signs))
    _abi.call('w8a8_swiglu_quantize', args)
    return res


def _epilogue_args(m, n, epilogue, row_scale, col_scale, bias, residual, out_dtype, out, device, gate=None,
                   gate_labels=None):
    if epilogue == EPI_INT32:
        if bias is not None or residual is not None:
            raise ValueError('raw int32 output takes no bias or residual')
        out = out if out is not None else torch.empty((m, n), dtype=torch.int32, device=device)
        if out.dtype != torch.int32 or tuple(out.shape) != (m, n) or out.stride(-1) != 1 or out.stride(0) < n:
            raise ValueError(f'out must be int32 [{m}, {n}] with unit column stride')
        _device(out)
        if out.device != device:
            raise ValueError('all tensors must be on the same device')
        if gate is not None:
            raise ValueError('raw int32 output takes no gate')
        return dict(row_scale=None, col_scale=None, col_scale_stride=0, bias=None, bias_dtype=0,
                    out_dtype=_abi.I32, residual=None, ldr=0, gate=None, gate_labels=None, ldg=0), out, ()
    if epilogue not in (EPI_ROW, EPI_COLUMN):
        raise ValueError('unknown epilogue')
    if out_dtype not in _OUT_DTYPES:
        raise ValueError('out_dtype must be float16, bfloat16 or float32')
    a = row_scale.to(torch.float32).reshape(-1).contiguous()
    if a.numel() != m:
        raise ValueError('row scale must have one entry per row')
    w, wstride = _scale_vec(col_scale, n, 'weight_scale')
    keep = [a, w]
    bias_dtype = 0
    if bias is not None:
        bias = bias.reshape(-1)
        if bias.dtype not in (torch.float16, torch.float32):
            bias = bias.float()
        bias = bias.contiguous()
        if bias.numel() != n:
            raise ValueError('bias must have one entry per output feature')
        bias_dtype = _abi.DTYPE_CODE[bias.dtype]
        keep.append(bias)
    ldr = 0
    if residual is not None:
        if out_dtype != torch.float16 or residual.dtype != torch.float16:
            raise ValueError('the fused residual add is FP16 only')
        residual = _rows_2d(residual)
        if residual.shape != (m, n):
            raise ValueError('residual must be [M, N]')
        ldr = residual.stride(0)
        keep.append(residual)
    ldg = 0
    if gate is not None:
        if residual is None:
            raise ValueError('the gate scales the residual update: residual required')
        gate = gate.to(torch.float32)
        if gate.ndim != 2 or gate.shape[1] != n or gate.stride(-1) != 1:
            gate = gate.reshape(-1, n).contiguous()
        if gate_labels is None or gate_labels.numel() != m:
            raise ValueError('gate_labels must give one gate-table row per output row')
        gate_labels = gate_labels.to(torch.int32).reshape(-1).contiguous()
        ldg = gate.stride(0)
        keep += [gate, gate_labels]
    elif gate_labels is not None:
        raise ValueError('gate_labels without a gate')
    if out is not None and (out.dtype != out_dtype or out.shape != (m, n) or out.stride(-1) != 1
                            or out.stride(0) < n):
        raise ValueError('out must be [M, N] of out_dtype with unit column stride')
    _device(a, w, bias, residual, gate, gate_labels, out)
    if a.device != device:
        raise ValueError('all tensors must be on the same device')
    out = out if out is not None else torch.empty((m, n), dtype=out_dtype, device=device)
    return dict(row_scale=a.data_ptr(), col_scale=w.data_ptr(), col_scale_stride=wstride,
                bias=_abi.ptr(bias), bias_dtype=bias_dtype, out_dtype=_abi.DTYPE_CODE[out_dtype],
                residual=_abi.ptr(residual), ldr=ldr, gate=_abi.ptr(gate), gate_labels=_abi.ptr(gate_labels),
                ldg=ldg), out, keep


_WORKSPACE_BYTES = {}


def _aligned16(t):
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _rope_epilogue(rope, m, device):
    """RopeEpilogue struct of a gemm() rope dict, and the tensors it points to."""
    heads, rot_dim = int(rope['heads']), int(rope['rot_dim'])
    freqs = rope['freqs']
    if freqs.dtype not in (torch.float16, torch.float32):
        raise ValueError('frequencies must be float16 or float32')
    if not (0 < rot_dim <= 128 and rot_dim % 2 == 0) or freqs.numel() != m * rot_dim * 2:
        raise ValueError('rope needs an even rot_dim <= 128 and freqs [M, rot_dim/2, 2, 2]')
    pairs = bool(rope.get('pairs', False))
    freqs = _aligned16(freqs.reshape((m, 2, rot_dim // 2, 2) if pairs else (m, rot_dim // 2, 2, 2)))
    gq = _aligned16(rope['q_gain'].to(torch.float32).reshape(-1))
    gk = _aligned16(rope['k_gain'].to(torch.float32).reshape(-1))
    _device(freqs, gq, gk)
    if freqs.device != device or gq.numel() != 128 or gk.numel() != 128:
        raise ValueError('rope tensors must be on the operands\' device, with 128-entry gains')
    args = _abi.RopeEpilogue(heads=heads, rot_dim=rot_dim, freq_dtype=_abi.DTYPE_CODE[freqs.dtype],
                             eps=float(rope.get('eps', 1e-6)), freq_layout=1 if pairs else 0, freqs=freqs.data_ptr(),
                             q_gain=gq.data_ptr(), k_gain=gk.data_ptr())
    return args, (freqs, gq, gk)


def gemm_workspace_bytes(m, n, k, device):
    """Split-K workspace bytes libw8a8 uses for an m x n x k GEMM on device
    (0 when the shape does not split); cached per shape and device."""
    key = (m, n, k, device.index)
    if key not in _WORKSPACE_BYTES:
        with torch.cuda.device(device):
            _WORKSPACE_BYTES[key] = int(_abi.load().w8a8_gemm_workspace_size(m, n, k))
    return _WORKSPACE_BYTES[key]


def gemm(q, weight, *, epilogue=EPI_INT32, row_scale=None, col_scale=None, bias=None, residual=None,
         out_dtype=torch.float16, out=None, workspace=None, gate=None, gate_labels=None, rope=None):
    """C = q @ weight.T on i8 MFMA with a fused epilogue.

    q int8 [M, K], weight int8 [N, K]. epilogue EPI_INT32 -> int32 [M, N];
    EPI_ROW -> out_dtype((C * a) * w [+ bias]); EPI_COLUMN ->
    out_dtype(C * (a * w) [+ bias]); residual (FP16 [M, N]) -> FP16
    residual + FP16 branch, and out may be the residual itself. gate (fp32
    [R, N]) with gate_labels (int32 [M], each row's table row) turns the
    residual add into fp16(fma(fp16(branch), gate[label], residual)).
    workspace: optional uint8 device tensor for split K; by default one of
    gemm_workspace_bytes() is allocated when the shape splits K (grids that
    would leave CUs idle). An empty tensor disables the split.
    rope: RMS-RoPE epilogue of a packed QKV projection, a dict with 'heads',
    'rot_dim', 'freqs' ([M, rot_dim/2, 2, 2] fp16/fp32 rotation matrices, or
    with 'pairs': True the [M, 2, rot_dim/2, 2] layout of
    rms_rope.pack_freqs), 'q_gain', 'k_gain' ([128]) and 'eps': the first
    2 * heads * 128 output columns (Q heads, then K heads) are stored
    normalized and rotated, bit-identical to rms_rope() of the plain FP16
    output; needs FP16 output without bias, residual or gate (K is never
    split).
    """
    q = _rows_2d(q)
    if weight.ndim != 2:
        raise ValueError('weight must be 2-D [N, K]')
    if weight.stride(-1) != 1:
        weight = weight.contiguous()
    if q.dtype != torch.int8 or weight.dtype != torch.int8:
        raise ValueError('int8 operands required')
    m, k = q.shape
    n = weight.shape[0]
    if weight.shape[1] != k:
        raise ValueError('Input and weight inner dimensions must match')
    if k % 16 or q.stride(0) % 16 or weight.stride(0) % 16:
        raise ValueError('K and the operand row strides must be multiples of 16')
    fields, out, keep = _epilogue_args(m, n, epilogue, row_scale, col_scale, bias, residual, out_dtype, out,
                                       q.device, gate, gate_labels)
    _device(q, weight, out)
    if m == 0 or n == 0:
        return out
    rope_args = None
    if rope is not None:
        rope_args, rope_keep = _rope_epilogue(rope, m, q.device)
        keep = (keep, rope_keep)
        workspace = torch.empty(0, dtype=torch.uint8, device=q.device)
    if workspace is None:
        nbytes = gemm_workspace_bytes(m, n, k, q.device)
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=q.device) if nbytes else None
    elif not workspace.is_cuda or workspace.device != q.device or not workspace.is_contiguous():
        raise ValueError('workspace must be a contiguous tensor on the operands\' device')
    ws_ptr = workspace.data_ptr() if workspace is not None and workspace.numel() else None
    ws_bytes = workspace.numel() * workspace.element_size() if ws_ptr else 0
    args = _abi.GemmArgs(epilogue=epilogue, a=q.data_ptr(), lda=q.stride(0), b=weight.data_ptr(),
                         ldb=weight.stride(0), m=m, n=n, k=k, out=out.data_ptr(), ldc=out.stride(0),
                         workspace=ws_ptr, workspace_bytes=ws_bytes, stream=_abi.stream_of(q),
                         rope=ctypes.pointer(rope_args) if rope_args is not None else None, **fields)
    _abi.call('w8a8_gemm', args)
    del keep, workspace
    return out


def dequantize(acc, row_scale, col_scale, *, epilogue=EPI_ROW, out_dtype=torch.float16, bias=None, residual=None,
               out=None, gate=None, gate_labels=None):
    """Standalone epilogue of an int32 accumulator [M, N]."""
    acc = _rows_2d(acc)
    _device(acc)
    if acc.dtype != torch.int32:
        raise ValueError('int32 accumulator required')
    if epilogue not in (EPI_ROW, EPI_COLUMN):
        raise ValueError('dequantize needs the ROW or COLUMN order')
    m, n = acc.shape
    fields, out, keep = _epilogue_args(m, n, epilogue, row_scale, col_scale, bias, residual, out_dtype, out,
                                       acc.device, gate, gate_labels)
    if m == 0 or n == 0:
        return out
    args = _abi.DequantArgs(epilogue=epilogue, acc=acc.data_ptr(), ldacc=acc.stride(0), m=m, n=n,
                            out=out.data_ptr(), ldc=out.stride(0), stream=_abi.stream_of(acc), **fields)
    _abi.call('w8a8_dequantize', args)
    del keep
    return out


ATTN_BLOCK_K = 128


def _row_strides(t):
    """(batch, head, token) element strides of a [B, H, N, 128] tensor whose
    rows the attention kernels can address in place (channels contiguous,
    16-byte aligned), or None."""
    esz = t.element_size()
    st = [0 if n == 1 else s for n, s in zip(t.shape, t.stride())]
    if st[3] != 1 or t.data_ptr() % 16 or any(s < 0 or (s * esz) % 16 for s in st[:3]):
        return None
    return tuple(st[:3])


def attention_prepare(q, k, v, *, sm_scale=None):
    """INT8 operands of the attention for q [B, H, Nq, 128], k, v [B, H, Nk,
    128] (fp16 or fp32), for the reference kernel's scheme with 128-key
    blocks. The inputs are read in place when their channels are contiguous
    and their strides 16-byte multiples (e.g. transposed views of a packed
    QKV projection), else from contiguous copies. Returns a dict with q8, qs
    (each row's group scale), k8, ks ([B, H, Nkp / 128, 4]: four group
    scales per block), vt8, vs, vsum ([B, H, Nkp / 128, 128]: 128 times each
    block's V code sums), all device tensors, the shape and sm_scale."""
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError('q, k, v must be [batch, heads, tokens, dim]')
    _device(q, k, v)
    b, h, nq, d = q.shape
    if k.shape != v.shape or k.shape[:2] != (b, h) or k.shape[3] != d:
        raise ValueError('q, k, v must share batch, heads and dim; k and v their shape')
    if d != 128:
        raise ValueError('INT8 attention supports 128-wide heads')
    if q.dtype not in (torch.float16, torch.float32) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError('q, k, v must all be float16 or all float32')
    nk = k.shape[2]
    if nq == 0 or nk == 0 or b * h == 0:
        raise ValueError('empty attention')
    if _row_strides(q) is None:
        q = q.contiguous()
    if _row_strides(k) is None:
        k = k.contiguous()
    if _row_strides(v) is None:
        v = v.contiguous()
    scale = float(d ** -0.5 if sm_scale is None else sm_scale)
    nkp = -(-nk // ATTN_BLOCK_K) * ATTN_BLOCK_K
    dev = q.device
    prep = dict(q8=torch.empty((b, h, nq, d), dtype=torch.int8, device=dev),
                qs=torch.empty((b, h, nq), dtype=torch.float32, device=dev),
                k8=torch.empty((b, h, nkp, d), dtype=torch.int8, device=dev),
                ks=torch.empty((b, h, nkp // ATTN_BLOCK_K, 4), dtype=torch.float32, device=dev),
                vt8=torch.empty((b, h, d, nkp), dtype=torch.int8, device=dev),
                vs=torch.empty((b, h, d), dtype=torch.float32, device=dev),
                vsum=torch.empty((b, h, nkp // ATTN_BLOCK_K, d), dtype=torch.int32, device=dev),
                shape=(b, h, nq, nk, d), sm_scale=scale)
    with torch.cuda.device(dev):
        nbytes = int(_abi.load().w8a8_attention_workspace_size(b, h, nk))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    args = _abi.AttnPrepareArgs(in_dtype=_abi.DTYPE_CODE[q.dtype], q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(),
                                b=b, h=h, nq=nq, nk=nk, d=d, sm_scale=scale, q_strides=_row_strides(q),
                                k_strides=_row_strides(k), v_strides=_row_strides(v),
                                q8=prep['q8'].data_ptr(), qs=prep['qs'].data_ptr(), k8=prep['k8'].data_ptr(),
                                ks=prep['ks'].data_ptr(), vt8=prep['vt8'].data_ptr(), vs=prep['vs'].data_ptr(),
                                vsum=prep['vsum'].data_ptr(), workspace=ws.data_ptr(), workspace_bytes=nbytes,
                                stream=_abi.stream_of(q))
    _abi.call('w8a8_attention_prepare', args)
    return prep


def attention(prep, *, out_dtype=torch.float16, out=None):
    """Attention output [B, H, Nq, 128] from attention_prepare()'s operands.
    ``out`` may be any [B, H, Nq, 128] view with contiguous channels and
    16-byte strides whose rows do not overlap (e.g. the transpose of a
    [B, Nq, H, 128] buffer, the layout the output projection reads)."""
    b, h, nq, nk, d = prep['shape']
    if out_dtype not in (torch.float16, torch.float32):
        raise ValueError('output must be float16 or float32')
    q8 = prep['q8']
    if out is None:
        out = torch.empty((b, h, nq, d), dtype=out_dtype, device=q8.device)
    elif out.shape != (b, h, nq, d) or out.dtype != out_dtype or _row_strides(out) is None:
        raise ValueError('out must be a [B, H, Nq, D] view of out_dtype with contiguous, 16-byte aligned rows')
    args = _abi.AttentionArgs(out_dtype=_abi.DTYPE_CODE[out_dtype], q8=q8.data_ptr(), qs=prep['qs'].data_ptr(),
                              k8=prep['k8'].data_ptr(), ks=prep['ks'].data_ptr(), vt8=prep['vt8'].data_ptr(),
                              vs=prep['vs'].data_ptr(), vsum=prep['vsum'].data_ptr(), b=b, h=h, nq=nq, nk=nk, d=d,
                              sm_scale=prep['sm_scale'], out=out.data_ptr(),
                              out_strides=_row_strides(out),
                              stream=_abi.stream_of(q8))
    _abi.call('w8a8_attention', args)
    return out
