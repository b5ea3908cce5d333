"""numpy restatement of the reference's W8A8 path arithmetic (test oracle).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product path.

Every float operation here is numpy float32 (IEEE binary32, round to nearest
even, no fused multiply-add), written in the exact order the reference
evaluates it; each function cites the reference lines it follows (paths are
relative to the reference repository root). bf16 tensors are carried as
uint16 bit patterns because numpy has no bfloat16.
"""
import numpy as np

F32 = np.float32
# fp32(1/127): the quantizer multiplies by this constant rather than dividing
# by 127 (patches/tilelang_row_quant.py:6-7,38 "max*float32(1/127)";
# benchmarks/verify_dit_p0a_p0c_local.py:140 clamp(max * (1./127.), min=1e-30)).
R127 = F32(1.0 / 127.0)
SCALE_FLOOR = F32(1e-30)
INV16 = F32(1.0 / 16.0)
GROUP = 256

# Cody-Waite constants and the degree-5 minimax polynomial of the Cephes
# single-precision exponential (S. L. Moshier, Cephes Math Library, expf.c).
_LOG2E = F32(1.44269504088896341)
_C1 = F32(0.693359375)
_C2 = F32(-2.12194440e-4)
_EXP_P = tuple(F32(c) for c in (1.9875691500e-4, 1.3981999507e-3, 8.3334519073e-3,
                                4.1665795894e-2, 1.6666665459e-1, 5.0000001201e-1))
_EXP_LO = F32(-104.0)   # exp(-104) is below the smallest fp32 subnormal / 2
_EXP_HI = F32(89.0)     # exp(89) overflows fp32


def _f32(x):
    return np.asarray(x, dtype=np.float32)


def to_bf16_bits(x):
    """fp32 -> bf16 bit pattern, round to nearest even (NaN stays NaN)."""
    x = _f32(x)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = np.isnan(x)
    out = rounded.astype(np.uint16)
    out[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return out


def from_bf16_bits(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def _to_f32(x, dtype):
    if dtype == 'bf16':
        return from_bf16_bits(x)
    return np.asarray(x).astype(np.float32)


def cast_out(y, dtype):
    """Storage cast of an fp32 result: 'f16', 'bf16' (uint16 bits) or 'f32'."""
    y = _f32(y)
    if dtype == 'f16':
        with np.errstate(over='ignore'):
            return y.astype(np.float16)
    if dtype == 'bf16':
        return to_bf16_bits(y)
    if dtype == 'f32':
        return y.copy()
    raise ValueError(dtype)


def quantize_rows(x, row_max=None):
    """Dynamic per-row absmax INT8 quantization.

    Follows benchmarks/verify_dit_p0a_p0c_local.py:140-147 (the reference's
    own torch restatement: scale = clamp(max * (1./127.), min=1e-30);
    q = round(x / scale).clamp(-128, 127).to(int8)) and the Kitchen contract
    quoted at patches/tilelang_row_quant.py:6-7 (max*fp32(1/127), floor
    1e-30, nearest-integer rounding, [-128,127] saturation). Division is
    IEEE (correctly rounded), rounding is half to even.
    ``row_max`` is an optional external absmax per row
    (patches/tilelang_row_quant.py:81-86, the global maximum over TP owners).
    Returns (q int8 [M,K], scale fp32 [M]).
    """
    x = _f32(x)
    if x.ndim != 2:
        raise ValueError('2-D input required')
    if row_max is None:
        amax = np.abs(x).max(axis=1) if x.shape[1] else np.zeros(x.shape[0], F32)
    else:
        amax = _f32(row_max).reshape(-1)
    with np.errstate(over='ignore'):
        scale = np.maximum(amax * R127, SCALE_FLOOR).astype(np.float32)
    with np.errstate(over='ignore', invalid='ignore', divide='ignore'):
        q = np.rint(x / scale[:, None])
    q = np.clip(q, -128, 127).astype(np.int8)
    return q, scale


def hadamard256():
    """Closed form of the regular-H4 ConvRot256 matrix (float64, scaled 1/16).

    H = (H4r)^{(x)4} / 16 with H4r = [[1,1,1,-1],[1,1,-1,1],[1,-1,1,1],
    [-1,1,1,1]]: H[i][j] = (-1)^{#base-4 digits d with i_d + j_d = 3} / 16.
    This is the matrix the butterfly of patches/tilelang_swiglu_quant.py:26-36
    applies (symmetric, H @ H = I). Used only to pin ``convrot256``.
    """
    idx = np.arange(GROUP)
    digits = np.stack([(idx >> (2 * d)) & 3 for d in range(4)], axis=-1)
    count = ((digits[:, None, :] + digits[None, :, :]) == 3).sum(-1)
    return np.where(count % 2 == 0, 1.0, -1.0) / 16.0


def convrot256(x, signs=None):
    """Regular-H4 ConvRot256 butterfly in fp32 over each 256-column group.

    Follows patches/tilelang_swiglu_quant.py:26-36 and :46: four stages with
    strides 1, 4, 16, 64; at output digit d the input at position 3-d is
    negated and the four inputs are summed as ((p + q) + r) + s in input
    order; after the last stage the values are multiplied by fp32(1/16).
    signs (optional, one +-1 per column; no counterpart in the reference,
    whose rotation has fixed signs): column j is negated first where
    signs[j] < 0, so the rotation is diag(signs) then H (a sign change is
    exact).
    """
    x = _f32(x)
    if x.shape[-1] % GROUP:
        raise ValueError('whole 256-column groups required')
    if signs is not None:
        s = np.asarray(signs).reshape(-1)
        if s.size != x.shape[-1]:
            raise ValueError('one sign per column required')
        x = np.where(s < 0, -x, x).astype(np.float32)
    shape = x.shape
    a = x.reshape(-1, GROUP).copy()
    for stage in range(4):
        stride = 4 ** stage
        v = a.reshape(a.shape[0], GROUP // (4 * stride), 4, stride)
        e0, e1, e2, e3 = v[:, :, 0, :], v[:, :, 1, :], v[:, :, 2, :], v[:, :, 3, :]
        out = np.empty_like(v)
        out[:, :, 0, :] = ((e0 + e1) + e2) + (-e3)
        out[:, :, 1, :] = ((e0 + e1) + (-e2)) + e3
        out[:, :, 2, :] = ((e0 + (-e1)) + e2) + e3
        out[:, :, 3, :] = (((-e0) + e1) + e2) + e3
        a = out.reshape(a.shape)
    return (a * INV16).reshape(shape)


def exp_f32(x):
    """This build's fp32 exponential (the same op sequence runs on the GPU).

    The reference calls CUDA ``expf`` inside its SwiGLU
    (patches/tilelang_swiglu_quant.py:22); that routine is not reproduced.
    This is the Cephes single-precision method (Cody-Waite reduction with the
    two-part ln2 C1 + C2, degree-5 minimax polynomial, Moshier's Cephes Math
    Library expf.c): inputs clamped to [-104, 89] (outside, fp32 exp is 0 or
    inf anyway), n = rne(x * log2 e) with one fp32 product, then the two
    reduction steps, the five Horner steps and p*z + r as fp32 fused
    multiply-adds (``fma_f32``, one rounding each; n*C1 is exact, so the first
    step equals x - n*C1), z = r*r and the final + 1 as fp32 operations, and
    the result scaled by ldexp.
    """
    x = _f32(x)
    with np.errstate(over='ignore', under='ignore', invalid='ignore'):
        x = np.fmin(np.fmax(x, _EXP_LO), _EXP_HI)
        n = np.rint(x * _LOG2E).astype(np.float32)
        r = fma_f32(-n, _C1, x)
        r = fma_f32(-n, _C2, r)
        z = r * r
        p = np.full_like(r, _EXP_P[0])
        for c in _EXP_P[1:]:
            p = fma_f32(p, r, c)
        y = fma_f32(p, z, r) + F32(1.0)
        return np.ldexp(y, n.astype(np.int32)).astype(np.float32)


def swiglu_f32(gate, up):
    """FP32 SwiGLU a = (g / (1 + exp(-g))) * u.

    Follows patches/tilelang_swiglu_quant.py:21-24: denominator = 1 +rn
    exp(-g); activated = g /rn denominator; A = activated *rn up.
    """
    g = _f32(gate)
    u = _f32(up)
    with np.errstate(over='ignore', invalid='ignore'):
        den = F32(1.0) + exp_f32(-g)
        act = g / den
        return (act * u).astype(np.float32)


def prepare_activation(x, convrot=True, x_dtype='f16', signs=None):
    """Column-path activation preparation: optional ConvRot256, then quantize.

    Follows patches/dit_column_linear.py:13-21: the rotation runs in x's
    dtype (the rotated tensor is x's dtype), then the per-row quantizer.
    Here the rotation is the regular-H4 butterfly of ``convrot256`` in fp32,
    rounded once to x's dtype. Parity unpinned: Kitchen's eager
    ``_rotate_activation`` is a GEMM against ``_build_hadamard`` whose fp32
    summation order is not available offline (comfy-kitchen 0.2.37 absent);
    both round the same exact sum, so they differ only where that sum lies
    within an fp32 rounding of an output-dtype midpoint.
    """
    xf = _to_f32(x, x_dtype)
    if convrot:
        r = convrot256(xf, signs)
        if x_dtype == 'f16':
            with np.errstate(over='ignore'):
                r = r.astype(np.float16).astype(np.float32)
        elif x_dtype == 'bf16':
            r = from_bf16_bits(to_bf16_bits(r))
        xf = r
    return quantize_rows(xf.reshape(-1, xf.shape[-1]))


def fc2_prologue(x, width=None, row_max=None, x_dtype='f16', return_rotated=False, signs=None):
    """Fused FC2 prologue: FP32 SwiGLU -> ConvRot256 -> row absmax -> quantize.

    Follows patches/tilelang_swiglu_quant.py:38-51 (stored phase: SwiGLU,
    butterfly, x1/16, per-group absmax), :67-92 (prepare: group max -> row
    max -> quantize) and patches/tilelang_row_quant.py:26-46 (scale =
    max(M * fp32(1/127), 1e-30), q = sat(rne(R / scale))) with IEEE division
    in place of the reference kernel's fast division, as in the reference's
    torch restatement (benchmarks/verify_dit_p0a_p0c_local.py:140-147).
    x: [M, 2W] with gate columns [0, W) and up columns [W, 2W).
    Returns (q, scale, group_max) or (q, scale, group_max, rotated).
    """
    xf = _to_f32(x, x_dtype)
    w = xf.shape[1] // 2 if width is None else width
    if w % GROUP or xf.shape[1] != 2 * w:
        raise ValueError('[M, 2W] input with W % 256 == 0 required')
    act = swiglu_f32(xf[:, :w], xf[:, w:])
    rot = convrot256(act, signs)
    gmax = np.abs(rot).reshape(rot.shape[0], w // GROUP, GROUP).max(-1)
    rmax = gmax.max(-1) if row_max is None else _f32(row_max).reshape(-1)
    q, scale = quantize_rows(rot, rmax)
    if return_rotated:
        return q, scale, gmax, rot
    return q, scale, gmax


def int_mm(q, w, w_f64=None):
    """INT32 C[m, n] = sum_k q[m, k] * w[n, k] (exact).

    Follows patches/parallel_int8.py:46-50 (torch._int_mm of the padded
    activations against weight.t()). Evaluated in float64 BLAS: every
    partial sum is an integer of magnitude <= K * 128 * 128 < 2^53, so the
    result is exact whatever the summation order. ``w_f64`` optionally
    supplies ``w.astype(float64)`` computed once by the caller.
    """
    q = np.asarray(q)
    w = np.asarray(w)
    if q.dtype != np.int8 or w.dtype != np.int8 or q.shape[1] != w.shape[1]:
        raise ValueError('int8 [M,K] x int8 [N,K] required')
    if q.shape[1] * 128 * 128 >= 2 ** 31:
        raise ValueError('K too large for exact int32 accumulation')
    wf = w.astype(np.float64) if w_f64 is None else w_f64
    acc = q.astype(np.float64) @ wf.T
    return acc.astype(np.int64).astype(np.int32)


def _col_scale(w, n):
    w = _f32(w).reshape(-1)
    if w.size == 1:
        return np.full(n, w[0], dtype=np.float32)
    if w.size != n:
        raise ValueError('scalar or per-channel weight scale required')
    return w


def dequantize_row(acc, a, w, dtype='f16', bias=None):
    """Row-order dequantization y = (f32(C) * a) * w [+ f32(bias)].

    Follows patches/parallel_int8.py:66-69 (left-to-right fp32 products,
    then the bias add, then one storage cast) and the fused transport
    epilogue's two rounded products (patches/tilelang_transport_p2.py:45-46).
    """
    acc = np.asarray(acc, dtype=np.int32)
    c = acc.astype(np.float32)
    y = (c * _f32(a).reshape(-1, 1)) * _col_scale(w, acc.shape[1])[None, :]
    if bias is not None:
        y = y + _to_f32(bias, 'f16' if np.asarray(bias).dtype == np.float16 else 'f32')[None, :]
    return cast_out(y, dtype)


def dequantize_column(acc, a, w, dtype='f16', bias=None):
    """Column-order dequantization y = f32(C) * (a * w) [+ f32(bias)].

    Follows patches/tilelang_column_epilogue.py:23-24 (scale = a *rn w, then
    value = f32(C) *rn scale) and patches/dit_column_linear.py:31-33; a bias
    is added after the products as in patches/parallel_int8.py:67-68.
    """
    acc = np.asarray(acc, dtype=np.int32)
    s = _f32(a).reshape(-1, 1) * _col_scale(w, acc.shape[1])[None, :]
    y = acc.astype(np.float32) * s
    if bias is not None:
        y = y + _to_f32(bias, 'f16' if np.asarray(bias).dtype == np.float16 else 'f32')[None, :]
    return cast_out(y, dtype)


def residual_add(x, branch):
    """x = f16(f32(x) + f32(branch)); patches/h3_tensor_flow.py:130-131."""
    with np.errstate(over='ignore'):
        return (np.asarray(x, np.float16).astype(np.float32)
                + np.asarray(branch, np.float16).astype(np.float32)).astype(np.float16)


def fma_f32(a, b, c):
    """fp32 fused multiply-add rounded once to nearest even: RN32(a*b + c).

    The GPU's v_fma_f32 / CUDA's __fmaf_rn. numpy has no fma, so: the float64
    product of two fp32 values is exact (48 significant bits); TwoSum gives
    the float64 sum s and its exact error e (s + e = a*b + c); rounding s to
    fp32 is then correct unless s sits exactly on an fp32 midpoint, where the
    sign of e decides (e == 0 keeps the tie to even).
    """
    a64 = _f32(a).astype(np.float64)
    b64 = _f32(b).astype(np.float64)
    c64 = _f32(c).astype(np.float64)
    with np.errstate(over='ignore', invalid='ignore'):
        prod = a64 * b64
        s = prod + c64
        bb = s - prod
        e = (prod - (s - bb)) + (c64 - bb)
        r = s.astype(np.float32)
        d = s - r.astype(np.float64)                      # exact: s and r are within half an fp32 ulp
        toward = np.where(d > 0, np.float32(np.inf), np.float32(-np.inf))
        other = np.nextafter(r, toward)                   # the fp32 neighbour on s's side of r
        mid = (r.astype(np.float64) + other.astype(np.float64)) * 0.5
        tie = (d != 0) & (s == mid) & (e != 0) & np.isfinite(s)
        out = np.where(tie & (np.sign(e) == np.sign(d)), other, r)
    return out.astype(np.float32)


def gated_residual_add(x, branch, gate, labels):
    """DiT gated residual update: f16(fma(f32(f16(branch)), gate[label], f32(x))).

    patches/tilelang_dit_fusion.py:72-75 (row_gate_kernel: the branch is
    rounded to FP16, then __fmaf_rn with the row's gate and the FP16
    residual); the eager route is h3_tensor_flow.gated_add (:145-152). gate is
    the fp32 table [R, N], labels the table row of every output row.
    """
    b16 = np.asarray(branch, np.float16).astype(np.float32)
    g = _f32(gate)[np.asarray(labels, np.int64)]
    with np.errstate(over='ignore'):
        return fma_f32(b16, g, np.asarray(x, np.float16).astype(np.float32)).astype(np.float16)


LANES = 64


def rms_sum_squares(x):
    """Per-row fp32 sum of squares in this build's fixed order.

    The reference sums the squares with TileLang's T.reduce_sum
    (patches/tilelang_dit_fusion.py:21-26: squares via __fmul_rn, zero past
    the width), whose order is the compiler's; this build fixes one: the
    row is cut into 16-element units, lane l of 64 adds, in order, the squares
    of units l, l+64, l+128, ... (elements in column order) to a partial
    starting at +0, then the 64 partials meet in an xor butterfly (offsets
    32, 16, 8, 4, 2, 1: p[l] = p[l] + p[l ^ off]). Addition is commutative
    in IEEE arithmetic, so every lane ends with the same total.
    """
    x = _f32(x)
    rows, cols = x.shape
    if cols % 16:
        raise ValueError('whole 16-element units required')
    units = cols // 16
    j = max(1, -(-units // LANES))
    sq = np.zeros((rows, j * LANES * 16), np.float32)
    with np.errstate(over='ignore'):
        sq[:, :cols] = x * x
    sq = sq.reshape(rows, j, LANES, 16)
    part = np.zeros((rows, LANES), np.float32)
    with np.errstate(over='ignore', invalid='ignore'):
        for jj in range(j):
            for i in range(16):
                part = part + sq[:, jj, :, i]
        lane = np.arange(LANES)
        for off in (32, 16, 8, 4, 2, 1):
            part = part + part[:, lane ^ off]
    return part[:, 0].copy()


def modulated_rms_norm(x, weight=None, shift=None, scale=None, labels=None, eps=1e-6, x_dtype='f16'):
    """DiT modulated RMSNorm in the fused kernel's fp32 operation order.

    patches/tilelang_dit_fusion.py:27-34 (norm_kernel): mean = ss * fp32(1/W);
    inv = rsqrtf(mean + eps); value = x * inv; gain = value * w;
    factor = 1 + scale[label]; y = x_dtype((gain * factor) + shift[label]),
    each step one fp32 rounding (__fmul_rn / __fadd_rn). Here rsqrtf (CUDA's
    approximate reciprocal square root, not reproduced) is replaced by a
    correctly rounded sqrt followed by a correctly rounded division, and the
    sum of squares follows ``rms_sum_squares``. The eager route
    (patches/h3_tensor_flow.py:134-142: F.rms_norm in fp32, then
    mul_(1 + scale).add_(shift) per segment) has the same sequence of
    operations. weight None: no gain; shift/scale None: plain RMSNorm.
    Returns x_dtype values (float16, or bf16 bit patterns as uint16).
    """
    xf = _to_f32(x, x_dtype)
    rows, cols = xf.shape
    ss = rms_sum_squares(xf)
    with np.errstate(over='ignore', invalid='ignore', divide='ignore'):
        mean = ss * F32(1.0 / cols)
        inv = F32(1.0) / np.sqrt(mean + F32(eps))
        y = xf * inv[:, None]
        if weight is not None:
            y = y * _f32(weight).reshape(1, -1)
        if shift is not None:
            lab = np.asarray(labels, np.int64).reshape(-1)
            factor = F32(1.0) + _f32(scale)[lab]
            y = y * factor
            y = y + _f32(shift)[lab]
    return cast_out(y.astype(np.float32), x_dtype)


def norm_quantize(x, weight=None, shift=None, scale=None, labels=None, eps=1e-6, x_dtype='f16', convrot=True,
                  round_rotated=True, signs=None):
    """Modulated RMSNorm followed by the column path's activation preparation.

    The composition of patches/tilelang_dit_fusion.py:10-36 (normalized rows
    stored in x's dtype) and patches/dit_column_linear.py:13-21 on them;
    round_rotated=False keeps the rotated values in fp32 instead.
    Returns (q int8, scale fp32 [M], y) with y the normalized rows.
    """
    y = modulated_rms_norm(x, weight, shift, scale, labels, eps, x_dtype)
    if convrot and not round_rotated:
        q, s = quantize_rows(convrot256(_to_f32(y, x_dtype), signs))
    else:
        q, s = prepare_activation(y, convrot, x_dtype, signs)
    return q, s, y


ROPE_DIM = 128


def head_sum_squares(x):
    """Sum of squares of each 128-element head vector in this build's order.

    The reference reduces with TileLang's T.reduce_sum
    (patches/tilelang_fp32_rms_rope.py:22-28, squares via __fmul_rn), whose
    order is the compiler's; this build fixes one: the vector is cut into 16
    slices of 8 elements, slice i adds its squares in order to a partial
    starting at +0, then the 16 partials meet in an xor butterfly (offsets 8,
    4, 2, 1). x: [..., 128] fp32.
    """
    x = _f32(x)
    sq = (x * x).astype(np.float32).reshape(*x.shape[:-1], 16, 8)
    part = np.zeros(sq.shape[:-1], np.float32)
    with np.errstate(over='ignore', invalid='ignore'):
        for i in range(8):
            part = part + sq[..., i]
        lane = np.arange(16)
        for off in (8, 4, 2, 1):
            part = part + part[..., lane ^ off]
    return part[..., 0].copy()


def rms_rope(packed, freqs, q_gain, k_gain, heads, rot_dim, eps=1e-6, in_dtype='f16', out_dtype='f16'):
    """Per-head FP32 RMS normalization and split-half RoPE of packed Q and K.

    patches/tilelang_fp32_rms_rope.py:27-43: per head vector, qr = rsqrtf(ss *
    fp32(1/dim) + eps); n = (x * qr) * gain; for d < rot_dim (pair p = d mod
    half, side s = d div half, partner = the other half) the output is
    __fmaf_rn(n[partner], F[p][s][1-s], n[d] * F[p][s][s]), else n[d]; each
    step one fp32 rounding, then the cast to the output dtype. rsqrtf
    (approximate) is replaced by a correctly rounded sqrt and division, and the
    sum of squares follows ``head_sum_squares``.
    packed: [rows, >= 2*heads*128] (Q heads, then K heads); freqs: [rows,
    rot_dim/2, 2, 2]. Returns (q, k), each [rows, heads, 128].
    """
    x = _to_f32(packed, in_dtype)
    rows = x.shape[0]
    width = heads * ROPE_DIM
    fr = _f32(np.asarray(freqs, np.float32)).reshape(rows, rot_dim // 2, 2, 2)
    half = rot_dim // 2
    outs = []
    for part, gain in ((x[:, :width], q_gain), (x[:, width:2 * width], k_gain)):
        v = part.reshape(rows, heads, ROPE_DIM)
        ss = head_sum_squares(v)
        with np.errstate(over='ignore', invalid='ignore', divide='ignore'):
            mean = ss * F32(1.0 / ROPE_DIM)
            inv = F32(1.0) / np.sqrt(mean + F32(eps))
            n = (v * inv[..., None]) * _f32(gain).reshape(1, 1, ROPE_DIM)
        n = n.astype(np.float32)
        out = n.copy()
        d = np.arange(rot_dim)
        side = (d >= half).astype(np.int64)
        pair = d - side * half
        other = np.where(side == 1, d - half, d + half)
        diag = fr[:, pair, side, side]              # [rows, rot_dim]
        offd = fr[:, pair, side, 1 - side]
        with np.errstate(over='ignore', invalid='ignore'):
            a = (n[:, :, :rot_dim] * diag[:, None, :]).astype(np.float32)
            out[:, :, :rot_dim] = fma_f32(n[:, :, other], np.broadcast_to(offd[:, None, :], a.shape), a)
        outs.append(cast_out(out, out_dtype))
    return outs[0], outs[1]


def quantize_weight(w):
    """Symmetric per-output-channel INT8 weights with fp32 scales.

    Not a reference function: the synthetic workloads quantize their fp32
    weights with the same per-row rule as the activations, so that every
    consumer of the weights sees identical bytes.
    """
    return quantize_rows(w)


def column_linear(x, wq, ws, convrot=True, x_dtype='f16', out_dtype='f16', bias=None, w_f64=None):
    """Column projection: prepare -> int_mm -> column-order dequantize.

    Follows patches/dit_column_linear.py:128-153 (_eager_column).
    """
    q, a = prepare_activation(x, convrot, x_dtype)
    return dequantize_column(int_mm(q, wq, w_f64), a, ws, out_dtype, bias)


def row_linear_fc2(x, wq, ws, residual=None, out_dtype='f16', x_dtype='f16', w_f64=None, gate=None, labels=None):
    """Row projection with the fused FC2 prologue (fused_stored route).

    Follows patches/tilelang_swiglu_quant.py:108-128 on one GPU (the SUM
    transport is the identity): prologue -> int_mm -> row-order dequantize;
    with a residual, the branch is cast to FP16 and added in FP32
    (patches/h3_tensor_flow.py:130-131), or with a gate table and row labels
    applied as the DiT gated update (gated_residual_add).
    """
    q, a, _ = fc2_prologue(x, x_dtype=x_dtype)
    acc = int_mm(q, wq, w_f64)
    if residual is None:
        return dequantize_row(acc, a, ws, out_dtype)
    branch = dequantize_row(acc, a, ws, 'f16')
    if gate is not None:
        return gated_residual_add(residual, branch, gate, labels)
    return residual_add(residual, branch)


def row_linear(x, wq, ws, residual=None, out_dtype='f16', x_dtype='f16', w_f64=None, gate=None, labels=None):
    """Row projection without an input activation (the DiT O projection).

    Follows patches/parallel_int8.py:26-43,72-94 on one GPU: ConvRot256 and
    the per-row quantizer in FP32 (the rotated values stay FP32, as
    patches/tilelang_dit_fusion.py:195-199 rotates value.float()), int_mm,
    the row-order dequantize, then the residual or gated update of
    row_linear_fc2 (the finish of patches/tilelang_dit_fusion.py:146-150).
    """
    xf = _to_f32(x, x_dtype)
    q, a = quantize_rows(convrot256(xf).reshape(-1, xf.shape[-1]))
    acc = int_mm(q, wq, w_f64)
    if residual is None:
        return dequantize_row(acc, a, ws, out_dtype)
    branch = dequantize_row(acc, a, ws, 'f16')
    if gate is not None:
        return gated_residual_add(residual, branch, gate, labels)
    return residual_add(residual, branch)


def row_partial(x, wq, row_max=None, swiglu=False, x_dtype='f16', w_f64=None):
    """One tensor-parallel rank's row projection before the SUM exchange.

    x is the rank's input: its K slice, or with ``swiglu`` its [gate_r |
    up_r] halves. Follows patches/tilelang_swiglu_quant.py:67-92 (prologue,
    then the quantizer with the MAX-exchanged row maximum) and, without
    SwiGLU, patches/tilelang_row_quant.py:114-146 / optimized_tp.py:53-87
    (FP32 ConvRot256 of the owned slice, external-maximum quantizer); then
    int_mm against the rank's weight columns (parallel_int8.py:86-91, before
    its all_reduce). ``row_max`` None uses the rank's own maximum.
    Returns (acc int32 [M, N], a fp32 [M]); the FP32 partial of the rank
    alone is dequantize_row(acc, a, ws, 'f32').
    """
    if swiglu:
        q, a, _ = fc2_prologue(x, row_max=row_max, x_dtype=x_dtype)
    else:
        xf = _to_f32(x, x_dtype)
        q, a = quantize_rows(convrot256(xf).reshape(-1, xf.shape[-1]), row_max)
    return int_mm(q, wq, w_f64), a


def rank_row_max(x, swiglu=False, x_dtype='f16'):
    """A rank's own row maximum, the MAX exchange's input (fp32 [M]): the
    absmax of ConvRot256(SwiGLU) or of the FP32 ConvRot256 of its slice."""
    xf = _to_f32(x, x_dtype)
    if swiglu:
        return fc2_prologue(xf, x_dtype='f32')[2].max(-1)
    return np.abs(convrot256(xf).reshape(-1, xf.shape[-1])).max(-1).astype(np.float32)


def ffn_block(h, w1q, ws1, w2q, ws2, residual, convrot=True, w1_f64=None, w2_f64=None, gate=None, labels=None):
    """DiT FFN block of the FP16-fix flow on one GPU.

    FC1 column projection (patches/tp_dit.py:356 -> dit_column_linear),
    then FC2 row projection with the fused SwiGLU/ConvRot256 prologue and the
    residual add (patches/tp_dit.py:360), or with the modulation gate table
    and row labels the DiT gated update; ws2 already carries the residual
    divisor (patches/h3_tensor_flow.py:82-103,114-127).
    """
    y1 = column_linear(h, w1q, ws1, convrot=convrot, w_f64=w1_f64)
    return row_linear_fc2(y1, w2q, ws2, residual=residual, w_f64=w2_f64, gate=gate, labels=labels)
