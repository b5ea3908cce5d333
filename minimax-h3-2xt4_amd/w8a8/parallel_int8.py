"""Quantization-preserving INT8 primitives (the reference's parallel_int8 API).

Same names, arguments and error behaviour as patches/parallel_int8.py, with
the arithmetic on libw8a8 (gfx950). One GPU: ``world_size`` must be 1 and
``comm`` is accepted but never used (the row-parallel SUM and the row-MAX
exchange are identities on one rank).
"""
import torch

from . import kernels

GROUPSIZE = 256


def _single_rank(world_size):
    if world_size != 1:
        raise ValueError('this build runs the W8A8 path on one GPU (world_size must be 1)')


def gather(x, comm, dim):
    """patches/parallel_int8.py:7-23 on one rank: the full tensor, offset 0."""
    world = comm.get_world_size() if comm is not None and comm.is_initialized() else 1
    _single_rank(world)
    return x, 0, x.shape[dim]


def quantize(x, groupsize=GROUPSIZE, input_act=None, input_act_weight=None, input_act_eps=0.0):
    """Row-wise INT8 with ConvRot, FP32 activation arithmetic.

    patches/parallel_int8.py:26-43: rotation is never silently skipped; with
    input_act='swiglu' the input is [M, 2W] (gate | up) and the FP32 SwiGLU
    runs before the rotation. Returns (q int8 [M, W], scale fp32 [M, 1]).
    The rotation stays in FP32 (the fused rotate-and-quantize route).
    """
    if groupsize != GROUPSIZE:
        raise ValueError('only the regular-H4 ConvRot256 group size is supported')
    if input_act_weight is not None or input_act_eps not in (0, 0.0):
        raise ValueError('input_act_weight / input_act_eps are not supported')
    flat = x.reshape(-1, x.shape[-1])
    if input_act == 'swiglu':
        if flat.dtype not in (torch.float16, torch.float32):
            flat = flat.float()
        res = kernels.swiglu_quantize(flat)
        return res['q'], res['scale']
    if input_act is not None:
        raise ValueError(f'unsupported input_act {input_act!r}')
    return kernels.quantize_rows(flat, convrot=True, round_rotated=False)


def int_mm(q, weight):
    """INT32 q @ weight.T (patches/parallel_int8.py:46-50); no padding needed."""
    return kernels.gemm(q, weight, epilogue=kernels.EPI_INT32)


def dequantize(accumulator, activation_scale, weight_scale, dtype, bias=None):
    """((f32(C) * a) * w) [+ bias] -> dtype (patches/parallel_int8.py:53-69).

    The order is the reference's eager order (two rounded products, then the
    bias add); it is not fused into an FMA.
    """
    return kernels.dequantize(accumulator, activation_scale, weight_scale, epilogue=kernels.EPI_ROW,
                              out_dtype=dtype, bias=bias)


def row_linear(x, weight, weight_scale, comm, world_size, groupsize=GROUPSIZE, input_act=None,
               bias=None, residual=None, residual_scale=None):
    """Row projection (patches/parallel_int8.py:72-94) on one rank.

    quantize (ConvRot, optional SwiGLU) -> INT32 GEMM -> row-order dequant
    fused into the GEMM epilogue; the optional legacy residual is
    addcmul(residual, out, residual_scale) after the storage cast.
    """
    _single_rank(world_size)
    q, scale = quantize(x, groupsize, input_act=input_act)
    out_dtype = x.dtype if x.dtype in (torch.float16, torch.bfloat16, torch.float32) else torch.float32
    out = kernels.gemm(q, weight, epilogue=kernels.EPI_ROW, row_scale=scale, col_scale=weight_scale, bias=bias,
                       out_dtype=out_dtype)
    del q
    out = out.reshape(*x.shape[:-1], weight.shape[0])
    if residual is not None:
        out = torch.addcmul(residual, out.to(x.dtype), residual_scale)
    return out.to(x.dtype)


def packed_rows(weight, scale, rank, world_size, components):
    """Component-wise column split (patches/parallel_int8.py:97-103)."""
    if weight.shape[0] % (components * world_size):
        raise ValueError('Packed components must divide evenly across ranks')
    chunks = weight.chunk(components, dim=0)
    scale_chunks = scale.chunk(components, dim=0)
    return (torch.cat([w.chunk(world_size, dim=0)[rank] for w in chunks], dim=0),
            torch.cat([s.chunk(world_size, dim=0)[rank] for s in scale_chunks], dim=0))
