"""External-maximum row quantization (the reference's tilelang_row_quant API).

Mirrors patches/tilelang_row_quant.py:81-86 (quantize) and :49-62 (maximum
over an owned slice). The reference kernel divides with a fast approximate
division; here division is always the IEEE quotient (``division`` is
accepted for API compatibility), which is what its torch restatement
computes.
"""
import torch

from . import kernels


def _check(rotated):
    if not rotated.is_cuda or rotated.dtype != torch.float32:
        raise ValueError('HIP FP32 input required')


def quantize(rotated, maximum, width=None, start=0, division='fast'):
    """q int8 [rows, width], scale fp32 [rows, 1] of rotated[:, start:start+width]."""
    _check(rotated)
    if division not in ('fast', 'rn'):
        raise ValueError('Unknown division mode')
    width = rotated.shape[1] if width is None else width
    if (rotated.ndim != 2 or not rotated.is_contiguous() or maximum.shape != (rotated.shape[0], 1)
            or maximum.dtype != torch.float32 or maximum.device != rotated.device):
        raise ValueError('Contiguous FP32 storage and matching global row maxima required')
    if rotated.shape[0] < 1 or width < 1 or start < 0 or start + width > rotated.shape[1]:
        raise ValueError('Invalid owned slice')
    if width % 16 or start % 4:
        raise ValueError('the owned slice must start on a 16-byte boundary and span a multiple of 16 columns')
    return kernels.quantize_rows(rotated[:, start:start + width], row_max=maximum)


def maximum(x, width=None, start=0):
    """Row absmax over the owned slice [start, start + width) -> fp32 [rows, 1]
    (the maximum phase of the quantize kernel: no codes are written)."""
    _check(x)
    width = x.shape[1] if width is None else width
    if x.ndim != 2 or x.shape[0] < 1 or start < 0 or width < 1 or start + width > x.shape[1]:
        raise ValueError('Invalid owned slice')
    if width % 16 or start % 4:
        raise ValueError('the owned slice must start on a 16-byte boundary and span a multiple of 16 columns')
    return kernels.row_absmax(x[:, start:start + width])
