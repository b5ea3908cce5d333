"""Column projections (the reference's dit_column_linear API).

Same names and arguments as patches/dit_column_linear.py. The activation is
rotated (regular-H4 ConvRot256, result in x's dtype) and quantized per row by
one libw8a8 kernel; the INT8 GEMM carries the column-order epilogue
fp16(f32(C) * (a * w)) so no int32 accumulator reaches HBM.
"""
import torch

from . import kernels

_BACKENDS = ('preallocated', 'cuda_int8_tilelang')


def _prepare_activation(x, convrot, convrot_groupsize):
    """Rotate (optional) and quantize rows; patches/dit_column_linear.py:13-21."""
    if convrot:
        if x.shape[-1] % convrot_groupsize:
            raise ValueError('ConvRot group size must divide input features')
        if convrot_groupsize != 256:
            raise ValueError('only the regular-H4 ConvRot256 group size is supported')
    return kernels.quantize_rows(x.reshape(-1, x.shape[-1]), convrot=bool(convrot), round_rotated=True)


def _weight_scale(weight, weight_scale, device):
    scale = weight_scale.to(device=device, dtype=torch.float32).reshape(-1)
    if scale.numel() not in (1, weight.shape[0]):
        raise ValueError('INT8 weight scale must be scalar or per-output-channel')
    return scale


def _column(codes, row_scale, weight, scale, out_dtype, bias=None):
    return kernels.gemm(codes, weight, epilogue=kernels.EPI_COLUMN, row_scale=row_scale, col_scale=scale,
                        bias=bias, out_dtype=out_dtype)


def shared_column_linears(x, projections, *, convrot=True, convrot_groupsize=256):
    """One activation preparation shared by several column projections.

    patches/dit_column_linear.py:70-96: returns None (caller keeps its own
    per-module path) when a projection does not match the input geometry.
    """
    flat = x.reshape(-1, x.shape[-1])
    for weight, weight_scale in projections:
        if weight.ndim != 2 or weight.shape[-1] != x.shape[-1] or weight_scale.numel() not in (1, weight.shape[0]):
            return None
    codes, row_scale = _prepare_activation(flat, convrot, convrot_groupsize)
    outputs = []
    for weight, weight_scale in projections:
        weight = weight.to(device=x.device).contiguous()
        scale = _weight_scale(weight, weight_scale, x.device)
        output = _column(codes, row_scale, weight, scale, x.dtype)
        outputs.append(output.reshape(*x.shape[:-1], weight.shape[0]))
    return tuple(outputs)


def column_linear(x, weight, weight_scale, *, convrot=True, convrot_groupsize=256, out_dtype=torch.float16,
                  backend='preallocated', p0_a1=False, bias=None):
    """Column projection; patches/dit_column_linear.py:99-125 / _eager_column :128-153.

    ``backend`` and ``p0_a1`` are accepted for API compatibility; every route
    runs the same fused kernels. ``bias`` (optional, [N]) is added after the
    column-order products.
    """
    if backend not in _BACKENDS:
        raise ValueError('Unknown column linear backend')
    if x.shape[-1] != weight.shape[-1]:
        raise ValueError('Input and weight inner dimensions must match')
    shape = x.shape
    weight = weight.to(device=x.device).contiguous()
    scale = _weight_scale(weight, weight_scale, x.device)
    codes, row_scale = _prepare_activation(x, convrot, convrot_groupsize)
    output = _column(codes, row_scale, weight, scale, out_dtype, bias)
    return output.reshape(*shape[:-1], weight.shape[0])


def column_linear_quantized(codes, row_scale, weight, weight_scale, *, out_dtype=torch.float16, bias=None):
    """Column projection of an activation already prepared (ConvRot256 and
    per-row INT8, e.g. by the fused modulated-norm kernel): the GEMM with the
    column-order epilogue of column_linear, without the preparation.
    """
    if codes.dtype != torch.int8 or codes.ndim != 2 or codes.shape[1] != weight.shape[-1]:
        raise ValueError('codes must be int8 [M, in_features]')
    weight = weight.to(device=codes.device).contiguous()
    scale = _weight_scale(weight, weight_scale, codes.device)
    return _column(codes, row_scale, weight, scale, out_dtype, bias)


def _eager_column(x, weight, weight_scale, *, convrot, convrot_groupsize, out_dtype, backend='preallocated'):
    return column_linear(x, weight, weight_scale, convrot=convrot, convrot_groupsize=convrot_groupsize,
                         out_dtype=out_dtype, backend=backend)
