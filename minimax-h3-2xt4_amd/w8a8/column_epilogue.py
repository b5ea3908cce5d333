"""Column-order INT32 dequantization (the reference's tilelang_column_epilogue API).

Mirrors patches/tilelang_column_epilogue.py:30-40: y = cast(f32(C) * (a * w)),
both FP32 products rounded, no reassociation.
"""
import torch

from . import kernels


def dequantize(accumulator, row_scale, weight_scale, out_dtype):
    if not accumulator.is_cuda or accumulator.dtype != torch.int32 or accumulator.ndim != 2:
        raise ValueError('HIP INT32 matrix required')
    rows, width = accumulator.shape
    if weight_scale.numel() not in (1, width):
        raise ValueError('Scalar or channel scale required')
    if out_dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError('Unsupported column dtype')
    return kernels.dequantize(accumulator, row_scale.reshape(rows, 1), weight_scale,
                              epilogue=kernels.EPI_COLUMN, out_dtype=out_dtype)
