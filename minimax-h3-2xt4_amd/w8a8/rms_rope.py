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


def pack_freqs(freqs):
    """The rotation matrices (1, S, 1, half, 2, 2) or [S, half, 2, 2] reordered
    for the QKV epilogue: [S, 2, half, 2] with entry [s][p] = (F[p][s][s],
    F[p][s][1 - s]) - the values a lane of side s needs, contiguous. A layout
    change only (no arithmetic); the DiT computes the matrices once per
    forward, so this runs once for all its blocks."""
    f = freqs.reshape(-1, freqs.shape[-3], 2, 2)
    side0 = torch.stack([f[:, :, 0, 0], f[:, :, 0, 1]], -1)
    side1 = torch.stack([f[:, :, 1, 1], f[:, :, 1, 0]], -1)
    return torch.stack([side0, side1], 1).contiguous()


def fused_qkv(x, weight, weight_scale, freqs, q_gain, k_gain, *, heads=28, dim=128, epsilon=1e-6, prepared=None,
              convrot=True, freqs_pairs=None):
    """The QKV projection followed by execute(), in one GEMM.

    patches/tp_dit.py:286-300 (qkv_proj, the split into q, k, v, then
    execute on the packed output) with the RMS-RoPE applied in the GEMM's
    epilogue to the FP16 values the projection would have stored, so the
    packed Q and K never make the round trip through HBM. x: [S, K] fp16
    activation (or prepared = (codes, row_scale), the ConvRot256 INT8
    activation of the fused modulated norm); weight int8 [3 * heads * dim, K]
    with its per-channel scale; freqs (1, S, 1, half, 2, 2); freqs_pairs, when
    given, is pack_freqs(freqs) (the faster layout for the epilogue). Returns
    (q, k, v), each a [S, heads, dim] view of the packed FP16 output; q and k
    equal execute(qkv_proj(x), ...) bit for bit, v equals the projection's V.
    """
    if dim != 128:
        raise ValueError('full 128-wide heads required')
    if prepared is None:
        codes, row_scale = kernels.quantize_rows(x.reshape(-1, x.shape[-1]), convrot=bool(convrot),
                                                 round_rotated=True)
    else:
        codes, row_scale = prepared
    rows = codes.shape[0]
    if weight.ndim != 2 or weight.shape[0] != 3 * heads * dim:
        raise ValueError('packed QKV weight of 3 * heads * dim rows required')
    if not (freqs.ndim == 6 and tuple(freqs.shape[:3]) == (1, rows, 1) and tuple(freqs.shape[-2:]) == (2, 2)
            and 0 < freqs.shape[-3] * 2 <= dim):
        raise ValueError('Packed QKV/frequency layout required')
    rot_dim = freqs.shape[-3] * 2
    weight = weight.to(device=codes.device).contiguous()
    scale = weight_scale.to(device=codes.device, dtype=torch.float32).reshape(-1)
    rope = {'heads': heads, 'rot_dim': rot_dim, 'freqs': freqs.reshape(rows, rot_dim // 2, 2, 2),
            'q_gain': q_gain, 'k_gain': k_gain, 'eps': float(epsilon)}
    if freqs_pairs is not None:
        if freqs_pairs.shape != (rows, 2, rot_dim // 2, 2):
            raise ValueError('freqs_pairs must be pack_freqs(freqs)')
        rope.update(freqs=freqs_pairs, pairs=True)
    qkv = kernels.gemm(codes, weight, epilogue=kernels.EPI_COLUMN, row_scale=row_scale, col_scale=scale,
                       out_dtype=torch.float16, rope=rope)
    q, k, v = qkv.split(heads * dim, dim=-1)
    return q.view(rows, heads, dim), k.view(rows, heads, dim), v.view(rows, heads, dim)
