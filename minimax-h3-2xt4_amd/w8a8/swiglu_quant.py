"""Fused FP32 SwiGLU / ConvRot256 FC2 prologue and the row projection using it.

Mirrors patches/tilelang_swiglu_quant.py (prepare, supported, row_linear).
On one GPU the row maximum is the global maximum, so 'fused_stored' runs as
one kernel (SwiGLU, butterfly, row max and quantization without an FP32
round trip); 'fused_recompute' runs the maximum phase and the
external-maximum quantize phase as two launches, as the reference does
around its MAX exchange.
"""
import torch

from . import kernels

_MODES = ('fused_stored', 'fused_recompute')


def prepare(x, comm=None, mode='fused_stored', *, arch=None, consume_input=False, p0_b=False):
    """(q int8 [M, W], scale fp32 [M, 1]) of x [.., 2W]; patches/tilelang_swiglu_quant.py:67-92."""
    if mode not in _MODES:
        raise ValueError(mode)
    if consume_input and mode != 'fused_stored':
        raise ValueError('P0-3 consumption requires fused_stored')
    width = x.shape[-1] // 2
    flat = x.reshape(-1, 2 * width)
    if mode == 'fused_stored':
        res = kernels.swiglu_quantize(flat)
    else:
        maximum = kernels.swiglu_quantize(flat, quantize=False, want_row_max=True)['row_max']
        res = kernels.swiglu_quantize(flat, row_max=maximum)
    if consume_input:
        # The prologue was the last reader of the FC1 output; release it.
        del flat
        x.set_()
    return res['q'], res['scale']


def supported(x, weight, weight_scale, world_size, groupsize):
    """Contract of the fused route; patches/tilelang_swiglu_quant.py:95-105 on one GPU."""
    width = x.shape[-1] // 2
    return (x.is_cuda and x.dtype in (torch.float16, torch.float32) and x.numel() > 0
            and x.shape[-1] == 2 * width and width % 256 == 0 and world_size == 1 and groupsize == 256
            and weight.ndim == 2 and weight.dtype == torch.int8 and weight.shape[1] == width
            and weight.device == x.device and weight_scale.dtype == torch.float32
            and weight_scale.is_contiguous() and weight_scale.numel() == weight.shape[0]
            and weight_scale.device == x.device)


def row_linear(x, weight, weight_scale, comm=None, *, mode='fused_stored', scaled_transport=False,
               finish_fn=None, consume_input=False, p0_b=False, residual=None, gate=None, gate_labels=None, out=None):
    """FC2 row projection; patches/tilelang_swiglu_quant.py:108-128 on one GPU.

    Without a residual it returns FP32 (C * a) * w, as the reference does
    before its caller's LoRA add. With ``residual`` (FP16 [M, N], the
    residual stream already divided by the tensor-flow divisor) the GEMM
    epilogue returns fp16(f32(residual) + f32(fp16(branch))), or with
    ``gate`` (fp32 [R, N]) and ``gate_labels`` (int32 [M]) the DiT gated
    update fp16(fma(fp16(branch), gate[label], residual)) of the reference's
    fused row_gate_kernel (patches/tilelang_dit_fusion.py:56-77). The scaled FP16
    transport is a two-rank codec; on one GPU the INT32 accumulator is exact
    and ``scaled_transport`` changes nothing. ``out`` (an extension of the
    reference's signature): a [M, N] tensor of the result dtype to write into,
    e.g. a row range of a larger buffer, instead of a new tensor.
    """
    if finish_fn is not None:
        raise ValueError('finish_fn belongs to the two-rank transport; pass residual= for the fused add')
    shape = x.shape
    q, scale = prepare(x, comm, mode, consume_input=consume_input, p0_b=p0_b)
    del x
    if out is not None:
        out = out.reshape(-1, weight.shape[0])
    if residual is None:
        out = kernels.gemm(q, weight, epilogue=kernels.EPI_ROW, row_scale=scale, col_scale=weight_scale,
                           out_dtype=torch.float32, out=out)
    else:
        out = kernels.gemm(q, weight, epilogue=kernels.EPI_ROW, row_scale=scale, col_scale=weight_scale,
                           out_dtype=torch.float16, residual=residual.reshape(-1, weight.shape[0]),
                           gate=gate, gate_labels=gate_labels, out=out)
    return out.reshape(*shape[:-1], weight.shape[0])
