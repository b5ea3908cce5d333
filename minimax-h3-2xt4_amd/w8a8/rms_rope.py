"""Packed QKV RMS-RoPE (the reference's tilelang_fp32_rms_rope API).

Same names and arguments as patches/tilelang_fp32_rms_rope.py:45-66:
``supported`` checks the packed layout and ``execute`` returns the normalized,
rotated Q and K as [rows, heads, dim]. The work runs in one libw8a8 kernel
(w8a8_rms_rope) on the caller's stream; V is not touched (the caller splits it
off the packed row as the reference does, patches/tp_dit.py:288-292).
"""
import torch

from . import kernels


def supported(packed, freqs, heads, dim):
    """Layout check of patches/tilelang_fp32_rms_rope.py:45-51 without the
    SM75 and 28-head pins: a 2-D contiguous fp16/fp32 packed row of 3 * heads *
    dim columns, dim = 128, and freqs of shape (1, rows, 1, half, 2, 2) with an
    even rotary prefix 0 < 2 * half <= dim, on the same device."""
    return (packed.is_cuda and packed.ndim == 2 and packed.dtype in (torch.float16, torch.float32)
            and packed.is_contiguous() and packed.shape[1] == 3 * heads * dim and dim == 128
            and freqs.device == packed.device and freqs.dtype in (torch.float16, torch.float32)
            and freqs.is_contiguous() and freqs.ndim == 6 and tuple(freqs.shape[:3]) == (1, packed.shape[0], 1)
            and tuple(freqs.shape[-2:]) == (2, 2) and 0 < freqs.shape[-3] * 2 <= dim)


def execute(packed, freqs, q_gain, k_gain, *, heads=28, dim=128, epsilon=1e-6, out_dtype=torch.float16):
    """patches/tilelang_fp32_rms_rope.py:54-66: (q, k), each [rows, heads, dim]."""
    if not supported(packed, freqs, heads, dim):
        raise ValueError('Packed QKV/frequency layout required')
    if out_dtype not in (torch.float16, torch.float32):
        raise ValueError('Explicit FP16/FP32 output required')
    rot_dim = freqs.shape[-3] * 2
    return kernels.rms_rope(packed, freqs.reshape(packed.shape[0], rot_dim // 2, 2, 2), q_gain, k_gain,
                            heads=heads, rot_dim=rot_dim, eps=float(epsilon), dim=dim, out_dtype=out_dtype)
