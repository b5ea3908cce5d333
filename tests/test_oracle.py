"""Pins of the CPU oracle: hand-computed answers, closed forms, invariants.

Each check is chosen so a plausible slip (a /127 instead of *fp32(1/127),
round-half-up, a wrong butterfly sign or summation order, swapped gate/up,
transposed operands, a swapped dequantization order) fails it.
"""
from fractions import Fraction

import numpy as np
import pytest

import oracle as o

F32 = np.float32


def f32_bits(x):
    return int(np.asarray(x, np.float32).view(np.uint32))


# ------------------------------------------------------------------ quantizer
def test_quantize_hand_computed_row():
    # amax 254: 254 * fp32(1/127) rounds to exactly 2.0, so q = rne(x / 2).
    x = np.array([[254.0, -127.0, 63.5, 0.0, 5.0, 7.0, -5.0, -7.0, 1.0, 3.0, -1.0, 0.5, 2.0, -2.0, 9.0, 11.0]],
                 np.float32)
    q, s = o.quantize_rows(x)
    assert s.tolist() == [2.0]
    # 127, -63.5->-64 (even), 31.75->32, 0, 2.5->2, 3.5->4, -2.5->-2, -3.5->-4,
    # 0.5->0, 1.5->2, -0.5->-0, 0.25->0, 1, -1, 4.5->4, 5.5->6
    assert q.tolist() == [[127, -64, 32, 0, 2, 4, -2, -4, 0, 2, 0, 0, 1, -1, 4, 6]]


def test_scale_is_product_with_fp32_reciprocal_not_division():
    # For amax 13 the two forms differ in the last bit.
    x = np.zeros((1, 16), np.float32)
    x[0, 3] = 13.0
    _, s = o.quantize_rows(x)
    assert f32_bits(s[0]) == 0x3DD1A346
    assert f32_bits(F32(13.0) / F32(127.0)) == 0x3DD1A347


def test_zero_row_scale_floor_and_codes():
    q, s = o.quantize_rows(np.zeros((2, 32), np.float32))
    assert f32_bits(s[0]) == f32_bits(F32(1e-30)) and f32_bits(s[1]) == f32_bits(F32(1e-30))
    assert not q.any()


def test_absmax_element_maps_to_pm127():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((64, 512)) * rng.uniform(1e-3, 1e3, (64, 1))).astype(np.float32)
    q, _ = o.quantize_rows(x)
    idx = np.abs(x).argmax(1)
    assert np.array_equal(np.abs(q[np.arange(64), idx]), np.full(64, 127))
    assert np.abs(q.astype(np.int32)).max() == 127


def test_external_max_saturates():
    x = np.array([[5.0, -5.0, 0.004, -0.006] + [0.0] * 12], np.float32)
    q, s = o.quantize_rows(x, row_max=np.array([1.27], np.float32))
    assert f32_bits(s[0]) == f32_bits(F32(1.27) * F32(1 / 127))
    assert q[0, :4].tolist() == [127, -128, 0, -1]


def test_quantize_matches_exact_rational_rounding():
    # Independent evaluation: exact rational x / s rounded half-even, against
    # the fp32 quotient the oracle rounds. They may differ only when the fp32
    # quotient itself rounds across a half-integer, which is rare.
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((8, 256)) * 3).astype(np.float32)
    q, s = o.quantize_rows(x)
    mism = 0
    for r in range(8):
        sr = Fraction(float(s[r]))
        for c in range(256):
            v = Fraction(float(x[r, c])) / sr
            fl = v.numerator // v.denominator
            rem = v - fl
            n = fl + (1 if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2) else 0)
            mism += int(max(-128, min(127, n)) != q[r, c])
    assert mism <= 2


# ------------------------------------------------------------------ ConvRot256
def test_hadamard_closed_form_properties():
    h = o.hadamard256()
    assert np.array_equal(h, h.T)
    assert np.array_equal(h @ h, np.eye(256))
    # Regular H4 (not Sylvester): entry (i=3, j=0) has one digit pair summing to 3.
    assert h[3, 0] == -1 / 16 and h[0, 3] == -1 / 16 and h[1, 2] == -1 / 16 and h[1, 1] == 1 / 16


def test_butterfly_equals_closed_form_on_integers():
    rng = np.random.default_rng(3)
    x = rng.integers(-2000, 2000, (9, 768)).astype(np.float32)
    ref = (x.reshape(-1, 256).astype(np.float64) @ o.hadamard256()).reshape(x.shape)
    assert np.array_equal(o.convrot256(x).astype(np.float64), ref)


def test_butterfly_unit_vectors_and_norm():
    eye = np.eye(256, dtype=np.float32)
    assert np.array_equal(o.convrot256(eye).astype(np.float64), o.hadamard256())
    rng = np.random.default_rng(4)
    x = rng.standard_normal((16, 1024)).astype(np.float32)
    r = o.convrot256(x)
    n0 = np.linalg.norm(x.reshape(-1, 256).astype(np.float64), axis=1)
    n1 = np.linalg.norm(r.reshape(-1, 256).astype(np.float64), axis=1)
    assert np.allclose(n0, n1, rtol=1e-6)


def test_signed_butterfly_equals_closed_form_and_inverts():
    # (x diag(s)) H exactly on integers (sums of 256 small integers / 16 are
    # exact in fp32); H H = I, so rotating again and re-applying the signs
    # gives x back, which a sign applied after the butterfly instead of
    # before would not.
    rng = np.random.default_rng(5)
    x = rng.integers(-2000, 2000, (7, 768)).astype(np.float32)
    s = rng.choice(np.array([-1, 1], np.int8), 768)
    ref = ((x.astype(np.float64) * s).reshape(-1, 256) @ o.hadamard256()).reshape(x.shape)
    r = o.convrot256(x, s)
    assert np.array_equal(r.astype(np.float64), ref)
    back = o.convrot256(r * 16) / 16
    assert np.array_equal(back * s, x)
    assert not np.array_equal(o.convrot256(x * s)[0], (o.convrot256(x) * s)[0])
    # all-positive signs are the unsigned rotation; a single negated column j
    # of the identity gives -H[j]
    assert np.array_equal(o.convrot256(x, np.ones(768, np.int8)), o.convrot256(x))
    eye = np.eye(256, dtype=np.float32)
    one = np.ones(256, np.int8)
    one[37] = -1
    assert np.array_equal(o.convrot256(eye, one).astype(np.float64)[37], -o.hadamard256()[37])
    assert np.array_equal(o.convrot256(eye, one)[36], o.convrot256(eye)[36])


def test_signed_prologues_rotate_before_quantizing():
    # The FC2 prologue and the column path with signs equal their unsigned
    # forms on inputs whose marked columns are negated first (SwiGLU is
    # applied before the rotation, so the signs act on its output).
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((5, 1024)) * 3).astype(np.float16)
    s = rng.choice(np.array([-1, 1], np.int8), 512)
    q, sc, gm = o.fc2_prologue(x, signs=s)
    act = o.swiglu_f32(x[:, :512].astype(np.float32), x[:, 512:].astype(np.float32))
    wq, ws = o.quantize_rows(o.convrot256(act * s))
    assert np.array_equal(q, wq) and np.array_equal(sc, ws)
    assert np.array_equal(gm, np.abs(o.convrot256(act * s)).reshape(5, 2, 256).max(-1))
    xs = (x[:, :512] * s).astype(np.float16)
    assert all(np.array_equal(a, b) for a, b in
               zip(o.prepare_activation(x[:, :512], True, 'f16', signs=s), o.prepare_activation(xs, True, 'f16')))


def test_butterfly_summation_order_left_to_right():
    # First quad [1e8, 1, -1e8, 1]: fp32 ((p+q)+r)+s gives -1, 2e8, 1, -2e8
    # (exact arithmetic would give 0, 2e8+2, 0, -2e8+2). The later stages only
    # spread these with signs (all other inputs are zero).
    x = np.zeros((1, 256), np.float32)
    x[0, :4] = [1e8, 1.0, -1e8, 1.0]
    r = o.convrot256(x)[0] * 16
    first = [-1.0, 2e8, 1.0, -2e8]
    for i in range(256):
        digits = [(i >> (2 * d)) & 3 for d in (1, 2, 3)]
        sign = -1.0 if sum(d == 3 for d in digits) % 2 else 1.0
        assert r[i] == F32(sign * first[i % 4]), i


# ------------------------------------------------------------------ exp / SwiGLU
def test_exp_accuracy_sweep():
    x = np.linspace(-87.0, 88.5, 400001).astype(np.float32)
    e = o.exp_f32(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.abs(e - ref) / np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert ulp.max() <= 2.0


def test_exp_special_values():
    assert o.exp_f32(np.float32(0.0)) == 1.0
    assert np.isinf(o.exp_f32(np.float32(89.0))) and np.isinf(o.exp_f32(np.float32(1000.0)))
    assert o.exp_f32(np.float32(-104.0)) < 1e-44 and o.exp_f32(np.float32(-1e4)) == 0.0
    assert abs(float(o.exp_f32(np.float32(1.0))) - np.e) < 3e-7


def test_swiglu_against_float64_and_special_values():
    rng = np.random.default_rng(5)
    g = (rng.standard_normal(200000) * 4).astype(np.float32)
    u = (rng.standard_normal(200000) * 4).astype(np.float32)
    a = o.swiglu_f32(g, u).astype(np.float64)
    gd, ud = g.astype(np.float64), u.astype(np.float64)
    ref = gd / (1 + np.exp(-gd)) * ud
    assert np.all(np.abs(a - ref) <= 4 * np.spacing(np.abs(ref).astype(np.float32)) + 1e-30)
    assert o.swiglu_f32(np.float32(0), np.float32(5)) == 0.0
    assert o.swiglu_f32(np.float32(100), np.float32(3)) == 300.0
    assert o.swiglu_f32(np.float32(-120), np.float32(3)) == 0.0
    # gate and up are not interchangeable
    assert o.swiglu_f32(np.float32(2), np.float32(-1)) != o.swiglu_f32(np.float32(-1), np.float32(2))


# ------------------------------------------------------------------ GEMM
def test_int_mm_brute_force():
    rng = np.random.default_rng(6)
    for m, n, k in ((1, 1, 16), (3, 5, 32), (13, 7, 64), (33, 17, 48)):
        a = rng.integers(-128, 128, (m, k)).astype(np.int8)
        b = rng.integers(-128, 128, (n, k)).astype(np.int8)
        ref = np.zeros((m, n), np.int64)
        for i in range(m):
            for j in range(n):
                ref[i, j] = sum(int(a[i, t]) * int(b[j, t]) for t in range(k))
        assert np.array_equal(o.int_mm(a, b), ref.astype(np.int32))


def test_int_mm_signed_extremes():
    k = 5120
    a = np.full((2, k), -128, np.int8)
    b = np.full((8, k), -128, np.int8)
    assert np.array_equal(o.int_mm(a, b), np.full((2, 8), k * 128 * 128, np.int32))
    b[1] = 127
    assert o.int_mm(a, b)[0, 1] == -128 * 127 * k


# ------------------------------------------------------------------ epilogues
def test_dequantize_reference_hand_example():
    # benchmarks/test_fp16_fc2_experiment.py:11-29: q=[1,-2,3,4], w=[2,3,-1,4],
    # accumulator 9, doubled by the fake SUM, scale .25, weight scale .125,
    # plus 1 -> fp16 1.5625.
    acc = o.int_mm(np.array([[1, -2, 3, 4]], np.int8), np.array([[2, 3, -1, 4]], np.int8)) * 2
    assert acc.tolist() == [[18]]
    y = o.dequantize_row(acc, np.array([0.25], np.float32), np.array([0.125], np.float32), 'f16',
                         bias=np.array([1.0], np.float32))
    assert y.dtype == np.float16 and y.tolist() == [[1.5625]]


def _f32_exact(x):
    return np.float32(float(x))


def test_row_and_column_orders_are_distinct_and_pinned():
    # Products of small integers and fp32 scales are exact in float64, so a
    # single cast rounds each product once.
    rng = np.random.default_rng(7)
    c = rng.integers(-(2 ** 20), 2 ** 20, (64, 48)).astype(np.int32)
    a = rng.uniform(1e-4, 1e-2, 64).astype(np.float32)
    w = rng.uniform(1e-4, 1e-2, 48).astype(np.float32)
    row = o.dequantize_row(c, a, w, 'f32')
    col = o.dequantize_column(c, a, w, 'f32')
    exp_row = np.empty_like(row)
    exp_col = np.empty_like(col)
    for i in range(64):
        for j in range(48):
            exp_row[i, j] = _f32_exact(float(_f32_exact(float(c[i, j]) * float(a[i]))) * float(w[j]))
            exp_col[i, j] = _f32_exact(float(c[i, j]) * float(_f32_exact(float(a[i]) * float(w[j]))))
    assert np.array_equal(row, exp_row)
    assert np.array_equal(col, exp_col)
    assert not np.array_equal(row, col)


def test_bias_added_after_products_and_fp16_cast():
    c = np.array([[1000, -3]], np.int32)
    y = o.dequantize_row(c, np.array([0.5], np.float32), np.array([0.25, 2.0], np.float32), 'f16',
                         bias=np.array([1.0, -0.5], np.float16))
    assert y.tolist() == [[126.0, -3.5]]
    big = o.dequantize_row(np.array([[2 ** 30]], np.int32), np.array([1.0], np.float32),
                           np.array([1.0], np.float32), 'f16')
    assert np.isinf(big[0, 0])


def test_bf16_rounding():
    x = np.array([1.0, 1.00390625, 1.005859375, -2.5, 3.0e38], np.float32)
    b = o.to_bf16_bits(x)
    # 1 + 2^-8 is a tie -> even (1.0); 1 + 1.5*2^-8 rounds up to 1 + 2^-7.
    assert o.from_bf16_bits(b).tolist()[:4] == [1.0, 1.0, 1.0078125, -2.5]


def test_residual_add_fp16():
    x = np.array([1.0, 2048.0], np.float16)
    br = np.array([0.0004883, 1.0], np.float16)
    out = o.residual_add(x, br)
    assert out.dtype == np.float16 and out.tolist() == [1.0, 2048.0]


# ------------------------------------------------------------------ composition
def test_fc2_prologue_against_float64_rotation():
    rng = np.random.default_rng(8)
    m, w = 6, 512
    x = (rng.standard_normal((m, 2 * w)) * 2).astype(np.float16)
    q, s, gmax, rot = o.fc2_prologue(x, return_rotated=True)
    g = x[:, :w].astype(np.float64)
    u = x[:, w:].astype(np.float64)
    act = g / (1 + np.exp(-g)) * u
    ref = (act.reshape(-1, 256) @ o.hadamard256()).reshape(m, w)
    assert np.allclose(rot, ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())
    assert np.array_equal(gmax, np.abs(rot).reshape(m, w // 256, 256).max(-1))
    ref_q = np.clip(np.rint(ref / s[:, None].astype(np.float64)), -128, 127)
    agree = (ref_q == q).mean()
    assert agree > 0.995 and np.abs(ref_q - q).max() <= 1
    # rotation preserves each group's norm (the 1/16 factor is present)
    n0 = np.linalg.norm(act.reshape(-1, 256), axis=1)
    n1 = np.linalg.norm(rot.reshape(-1, 256).astype(np.float64), axis=1)
    assert np.allclose(n0, n1, rtol=1e-5)


def test_fc2_prologue_external_max():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((3, 512)).astype(np.float16)
    q1, s1, g1 = o.fc2_prologue(x)
    q2, s2, _ = o.fc2_prologue(x, row_max=g1.max(-1) * 2)
    assert np.array_equal(s2, np.maximum(g1.max(-1) * 2 * o.R127, o.SCALE_FLOOR))
    assert np.abs(q2.astype(int)).max() <= 64


def test_column_path_rounds_rotation_to_input_dtype():
    rng = np.random.default_rng(10)
    x = rng.standard_normal((4, 256)).astype(np.float16)
    q16, s16 = o.prepare_activation(x, convrot=True, x_dtype='f16')
    rot16 = o.convrot256(x.astype(np.float32)).astype(np.float16).astype(np.float32)
    assert np.array_equal(s16, np.abs(rot16).max(1) * o.R127)
    qn, sn = o.prepare_activation(x, convrot=False, x_dtype='f16')
    assert np.array_equal(qn, o.quantize_rows(x.astype(np.float32))[0])


def test_end_to_end_linear_close_to_float64():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((32, 512)).astype(np.float16)
    w = (rng.standard_normal((64, 512)) * 0.02).astype(np.float32)
    wq, ws = o.quantize_weight(w)
    y = o.column_linear(x, wq, ws, convrot=False).astype(np.float64)
    ref = x.astype(np.float64) @ w.T.astype(np.float64)
    assert np.abs(y - ref).max() / np.abs(ref).max() < 0.03
    with pytest.raises(ValueError):
        o.int_mm(np.zeros((2, 8), np.int8), np.zeros((3, 16), np.int8))


# ------------------------------------------------------------------ fused multiply-add and the DiT gate
def _rn32_exact(value):
    """Round an exact Fraction to fp32 (nearest, ties to even) by brute force."""
    from fractions import Fraction
    f = np.float32(float(value))
    cands = [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
    dist = [abs(Fraction(float(c)) - value) for c in cands]
    best = [c for c, d in zip(cands, dist) if d == min(dist)]
    if len(best) > 1:
        best = [c for c in best if (np.asarray(c, np.float32).view(np.uint32) & 1) == 0]
    return best[0]


def test_fma_f32_matches_exact_rational_rounding():
    from fractions import Fraction
    rng = np.random.default_rng(7)
    a = (rng.standard_normal(3000) * 10.0 ** rng.integers(-8, 8, 3000)).astype(np.float32)
    b = (rng.standard_normal(3000) * 10.0 ** rng.integers(-8, 8, 3000)).astype(np.float32)
    c = (rng.standard_normal(3000) * 10.0 ** rng.integers(-8, 8, 3000)).astype(np.float32)
    got = o.fma_f32(a, b, c)
    for i in range(3000):
        want = _rn32_exact(Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i])))
        assert got[i] == want, (i, a[i], b[i], c[i], got[i], want)


def test_fma_f32_single_rounding_and_midpoint_correction():
    one = np.float32(1 + 2.0 ** -12)
    # fused keeps the 2^-24 term that the unfused product rounds away (tie to even)
    assert o.fma_f32(one, one, np.float32(-1.0)) == np.float32(2.0 ** -11 + 2.0 ** -24)
    assert (one * one) - np.float32(1.0) == np.float32(2.0 ** -11)
    # a*b = 1 + 2^-11 + 2^-24 is an fp32 midpoint; the float64 sum loses +-2^-80,
    # which must still decide the direction
    assert o.fma_f32(one, one, np.float32(2.0 ** -80)) == np.float32(1 + 2.0 ** -11 + 2.0 ** -23)
    assert o.fma_f32(one, one, np.float32(-(2.0 ** -80))) == np.float32(1 + 2.0 ** -11)
    assert o.fma_f32(one, one, np.float32(0.0)) == np.float32(1 + 2.0 ** -11)   # exact tie: even


def test_gated_residual_add_composition():
    x = np.array([[1.0, -2.0], [0.5, 3.0]], np.float16)
    branch = np.array([[0.25, 1.0], [2.0, -1.0]], np.float32)
    gate = np.array([[2.0, 0.5], [-1.0, 4.0], [0.0, 0.0]], np.float32)
    labels = np.array([1, 0])
    got = o.gated_residual_add(x, branch, gate, labels)
    want = np.array([[1.0 - 0.25, -2.0 + 4.0], [0.5 + 4.0, 3.0 - 0.5]], np.float16)
    assert np.array_equal(got, want)
    # the branch is rounded to FP16 before the FMA (tilelang_dit_fusion.py:72-75)
    b = np.array([[1 + 2.0 ** -12]], np.float32)
    assert o.gated_residual_add(np.zeros((1, 1), np.float16), b, np.ones((1, 1), np.float32), [0])[0, 0] == 1.0


# ------------------------------------------------------- modulated RMSNorm
def test_rms_sum_squares_exact_on_integer_squares():
    rng = np.random.default_rng(11)
    x = rng.integers(-8, 9, (7, 3072)).astype(np.float32)   # every partial sum < 2^24: any order is exact
    assert np.array_equal(o.rms_sum_squares(x), (x.astype(np.int64) ** 2).sum(1).astype(np.float32))
    x = rng.integers(-8, 9, (3, 336 * 16)).astype(np.float32)  # 336 units: a partial last lane block
    assert np.array_equal(o.rms_sum_squares(x), (x.astype(np.int64) ** 2).sum(1).astype(np.float32))


def test_rms_sum_squares_lane_order_known_answer():
    # Lane 0 owns units 0 and 64: its 16 unit-64 squares of 1 are absorbed one
    # at a time by 2^24 (2^24 + 1 rounds to even); lanes 1..63 hold 16 each and
    # meet lane 0 in the butterfly: 2^24 + 16 + 32 + 64 + 128 + 256 + 512.
    x = np.zeros((1, 2048), np.float32)
    x[0, 0] = 4096.0
    x[0, 16:64 * 16] = 1.0
    x[0, 64 * 16:65 * 16] = 1.0
    assert o.rms_sum_squares(x)[0] == np.float32(2 ** 24 + 1008)
    # A plain left-to-right sum would give 2^24, the exact sum 2^24 + 1024.


def test_rms_sum_squares_butterfly_offsets_descend():
    # Partials: lane 0 = 2^24, lane 32 = 3, the others 1. Offset 32 first:
    # 2^24 + 3 is a tie and rounds to 2^24 + 4; then + 2 + 4 + 8 + 16 + 32.
    x = np.zeros((1, 1024), np.float32)
    x[0, 0] = 4096.0
    for lane in range(1, 64):
        x[0, 16 * lane] = 1.0
    x[0, 16 * 32:16 * 32 + 3] = 1.0
    assert o.rms_sum_squares(x)[0] == np.float32(2 ** 24 + 66)
    # Ascending offsets would absorb lane 1's 1 first (2^24 + 1 -> 2^24).


def test_rms_sum_squares_error_bound():
    rng = np.random.default_rng(12)
    x = (rng.standard_normal((16, 5376)) * 3).astype(np.float16).astype(np.float32)
    exact = (x.astype(np.float64) ** 2).sum(1)
    n = 6 * 16 + 6   # terms per lane plus butterfly stages
    assert np.all(np.abs(o.rms_sum_squares(x) - exact) <= n * 2.0 ** -24 * exact)


def test_float32_sqrt_and_reciprocal_are_correctly_rounded():
    # Rounding the float64 result once to fp32 is correctly rounded for sqrt
    # and division (53 >= 2*24 + 2), so numpy's float32 ops must agree.
    rng = np.random.default_rng(13)
    d = np.exp(rng.uniform(-80, 80, 200000)).astype(np.float32)
    r = np.sqrt(d)
    assert np.array_equal(r, np.sqrt(d.astype(np.float64)).astype(np.float32))
    assert np.array_equal(np.float32(1.0) / r, (1.0 / r.astype(np.float64)).astype(np.float32))


def test_modulated_norm_constant_rows_are_unit():
    for cols in (1024, 4096):
        x = np.zeros((4, cols), np.float16)
        x[0], x[1], x[2], x[3] = 0.5, -2.0, 0.0625, 8.0
        y = o.modulated_rms_norm(x, eps=0.0)
        assert np.array_equal(y, np.sign(x.astype(np.float32)).astype(np.float16))


def test_modulated_norm_scale_minus_one_selects_shift_row():
    rng = np.random.default_rng(14)
    x = rng.standard_normal((6, 512)).astype(np.float16)
    w = rng.uniform(0.5, 2, 512).astype(np.float32)
    shift = rng.standard_normal((5, 512)).astype(np.float32)
    scale = np.full((5, 512), -1.0, np.float32)
    labels = np.array([4, 0, 2, 2, 1, 3], np.int32)
    y = o.modulated_rms_norm(x, w, shift, scale, labels, eps=1e-6)
    assert np.array_equal(y, shift[labels].astype(np.float16))


def test_modulated_norm_against_torch_rms_norm():
    import torch
    rng = np.random.default_rng(15)
    x = (rng.standard_normal((9, 3072)) * 4).astype(np.float16)
    w = rng.uniform(0.5, 1.5, 3072).astype(np.float32)
    shift = (rng.standard_normal((3, 3072)) * 0.1).astype(np.float32)
    scale = (rng.standard_normal((3, 3072)) * 0.1).astype(np.float32)
    labels = np.array([0, 0, 1, 1, 1, 2, 2, 0, 1], np.int32)
    eps = 1e-6 / 512 ** 2
    y = o.modulated_rms_norm(x, w, shift, scale, labels, eps=eps)
    h = torch.nn.functional.rms_norm(torch.from_numpy(x).double(), (3072,), torch.from_numpy(w).double(), eps)
    h = h * (1 + torch.from_numpy(scale[labels]).double()) + torch.from_numpy(shift[labels]).double()
    ref = h.numpy()
    # fp16 output rounding (2^-11 relative) plus a few fp32 roundings.
    assert np.all(np.abs(y.astype(np.float64) - ref) <= 2.0 ** -11 * np.abs(ref) + 1e-6)
    yb = o.from_bf16_bits(o.modulated_rms_norm(o.to_bf16_bits(x.astype(np.float32)), w, shift, scale, labels,
                                               eps=eps, x_dtype='bf16'))
    xb = o.from_bf16_bits(o.to_bf16_bits(x.astype(np.float32))).astype(np.float64)
    hb = torch.nn.functional.rms_norm(torch.from_numpy(xb), (3072,), torch.from_numpy(w).double(), eps)
    refb = (hb * (1 + torch.from_numpy(scale[labels]).double()) + torch.from_numpy(shift[labels]).double()).numpy()
    assert np.all(np.abs(yb - refb) <= 2.0 ** -8 * np.abs(refb) + 1e-6)


def test_norm_quantize_composition():
    rng = np.random.default_rng(16)
    x = rng.standard_normal((5, 512)).astype(np.float16)
    shift = np.zeros((2, 512), np.float32)
    scale = np.full((2, 512), -1.0, np.float32)
    shift[1, :] = 0.25
    labels = np.array([0, 1, 1, 0, 1], np.int32)
    q, s, y = o.norm_quantize(x, None, shift, scale, labels, eps=1e-6, convrot=False)
    # rows on label 0 are all zero (scale floor, codes 0); label 1 rows are constant 0.25 -> 127
    assert np.array_equal(s[labels == 0], np.full(2, o.SCALE_FLOOR))
    assert np.all(q[labels == 0] == 0) and np.all(q[labels == 1] == 127)
    q2, s2, y2 = o.norm_quantize(x, None, shift, scale, labels, eps=1e-6, convrot=True)
    # the rotated constant rows quantize like the rotation of a constant 0.25 row
    r = o.convrot256(np.full((1, 512), 0.25, np.float32))
    assert np.array_equal(q2[1], o.quantize_rows(r)[0][0])


# ------------------------------------------------------------ RMS-RoPE
def _rope_freqs(angles):
    c, s = np.cos(angles), np.sin(angles)
    return np.stack([np.stack([c, -s], -1), np.stack([s, c], -1)], -2).astype(np.float32)


def test_head_sum_squares_exact_and_order():
    rng = np.random.default_rng(21)
    x = rng.integers(-20, 21, (6, 128)).astype(np.float32)
    assert np.array_equal(o.head_sum_squares(x), (x.astype(np.int64) ** 2).sum(-1).astype(np.float32))
    # Slice 0 holds 2^24 then seven squares of 1 (absorbed one at a time); slices
    # 1..15 hold 8 each; offset 8 meets slice 8 first: 2^24 + 8 + 16 + 32 + 64.
    x = np.ones((1, 128), np.float32)
    x[0, 0] = 4096.0
    assert o.head_sum_squares(x)[0] == np.float32(2 ** 24 + 120)   # exact sum: 2^24 + 127


def test_rms_rope_identity_frequencies_are_the_norm():
    rng = np.random.default_rng(22)
    rows, heads, rot = 3, 2, 96
    p = (rng.standard_normal((rows, 3 * heads * 128)) * 2).astype(np.float16)
    gq = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    gk = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    f = _rope_freqs(np.zeros((rows, rot // 2)))
    q, k = o.rms_rope(p, f, gq, gk, heads, rot, eps=1e-6, out_dtype='f32')
    x = p.astype(np.float32)[:, :2 * heads * 128].reshape(rows, 2, heads, 128)
    inv = np.float32(1) / np.sqrt(o.head_sum_squares(x) * np.float32(1 / 128) + np.float32(1e-6))
    want_q = (x[:, 0] * inv[:, 0, :, None]) * gq
    want_k = (x[:, 1] * inv[:, 1, :, None]) * gk
    assert np.array_equal(q, want_q) and np.array_equal(k, want_k)


def test_rms_rope_quarter_turn_swaps_halves():
    rng = np.random.default_rng(23)
    rows, heads, rot = 2, 2, 96
    p = rng.standard_normal((rows, 3 * heads * 128)).astype(np.float16)
    g = np.ones(128, np.float32)
    f = _rope_freqs(np.full((rows, rot // 2), np.pi / 2))
    f = np.round(f)                                   # exactly [[0, -1], [1, 0]]
    base, _ = o.rms_rope(p, _rope_freqs(np.zeros((rows, rot // 2))), g, g, heads, rot, out_dtype='f32')
    q, _ = o.rms_rope(p, f, g, g, heads, rot, out_dtype='f32')
    h = rot // 2
    assert np.array_equal(q[..., :h], -base[..., h:rot])
    assert np.array_equal(q[..., h:rot], base[..., :h])
    assert np.array_equal(q[..., rot:], base[..., rot:])


def test_rms_rope_power_of_two_scale_invariance_and_float64():
    import torch
    rng = np.random.default_rng(24)
    rows, heads, rot = 4, 3, 96
    p = rng.standard_normal((rows, 3 * heads * 128)).astype(np.float32)
    gq = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    gk = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    f = _rope_freqs(rng.uniform(0, 2 * np.pi, (rows, rot // 2)))
    q, k = o.rms_rope(p, f, gq, gk, heads, rot, eps=0.0, in_dtype='f32', out_dtype='f32')
    q2, k2 = o.rms_rope(p * np.float32(8), f, gq, gk, heads, rot, eps=0.0, in_dtype='f32', out_dtype='f32')
    assert np.array_equal(q, q2) and np.array_equal(k, k2)
    x = torch.from_numpy(p).double()[:, :heads * 128].reshape(rows, heads, 128)
    n = torch.nn.functional.rms_norm(x, (128,), torch.from_numpy(gq).double(), 0.0)
    ft = torch.from_numpy(f).double()
    lo, hi = n[..., :rot // 2], n[..., rot // 2:rot]
    out = n.clone()
    out[..., :rot // 2] = ft[:, None, :, 0, 0] * lo + ft[:, None, :, 0, 1] * hi
    out[..., rot // 2:rot] = ft[:, None, :, 1, 0] * lo + ft[:, None, :, 1, 1] * hi
    assert np.max(np.abs(q - out.numpy())) < 4e-6 * np.max(np.abs(out.numpy()))


# ------------------------------------------------------------ INT8 attention
from oracle import int8_attention as oa  # noqa: E402


def test_attention_oracle_layout_and_prepare_pins():
    perm = oa.perm32()
    assert sorted(perm.tolist()) == list(range(32))
    assert perm[:8].tolist() == [0, 1, 2, 3, 8, 9, 10, 11] and perm[16:20].tolist() == [4, 5, 6, 7]
    # integer keys: the chunked fp32 mean is exact
    k = np.arange(2 * 300 * 128, dtype=np.float32).reshape(1, 2, 300, 128) % 7 - 3
    assert np.array_equal(oa.key_mean(k), k.astype(np.float64).mean(2).astype(np.float32))
    rng = np.random.default_rng(1)
    q = rng.standard_normal((1, 1, 5, 128)).astype(np.float32)
    v = rng.standard_normal((1, 1, 300, 128)).astype(np.float32)
    pr = oa.kitchen_prepare(q, k[:, :1], v, cta_k=oa.GPU_CTA_K)
    g = oa.gpu_operands(pr)
    # each Q group's absmax element maps to +-127 (rows 0..4 are their own
    # groups); the scale is amax / 127 + 1e-7 in fp32
    assert np.all(np.abs(g['q8']).max(-1) == 127)
    assert np.array_equal(g['qs'], (np.abs(q).max(-1) / np.float32(127) + np.float32(1e-7)).astype(np.float32))
    # centred keys (integers minus the exact mean), four scales per 128-key
    # block, zero padding past nk
    assert g['k8'].shape == (1, 1, 384, 128) and not g['k8'][:, :, 300:].any()
    assert g['ks'].shape == (1, 1, 3, 4)
    kc = k[:, :1] - pr['kmean'][:, :, None, :]
    amax = np.abs(kc[0, 0, [128 + 8 * t + 4 + e for t in range(16) for e in (0, 1)]]).max()
    assert g['ks'][0, 0, 1, 2] == np.float32(amax / np.float32(127) + np.float32(1e-7))
    # the last block's groups hold keys 256..299 and zero padding: every scale
    # stays positive, so the out-of-bounds score masks the padded keys
    assert np.all(g['ks'] > 0)
    # V^T holds key perm(p) of each 32-key group at position p
    assert np.array_equal(g['vt8'][0, 0, :, 32 + 5], pr['v8'][0, 0, 32 + perm[5], :])
    # 128 times each block's code sums, per channel
    assert np.array_equal(g['vsum'][0, 0, 2], 128 * pr['v8'][0, 0, 256:384].astype(np.int64).sum(0))
    # round half away from zero as the restated quantizer takes it in fp32
    assert oa._round_half_away(np.float32([0.5, -0.5, 1.5, -2.5, 0.49999997])).tolist() == [1, -1, 2, -3, 1]


def test_attention_oracle_against_closed_forms():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((1, 2, 40, 128)).astype(np.float32)
    k = rng.standard_normal((1, 2, 300, 128)).astype(np.float32)
    v = rng.standard_normal((1, 2, 300, 128)).astype(np.float32)
    out = oa.kitchen_attention(oa.kitchen_prepare(q, k, v, cta_k=oa.GPU_CTA_K)).astype(np.float64)
    exact = oa.reference_attention(q, k, v)
    cos = (out * exact).sum() / np.sqrt((out * out).sum() * (exact * exact).sum())
    assert cos > 0.9995
    # a wrong softmax scale fails the comparison with exact attention
    wrong = oa.kitchen_attention(oa.kitchen_prepare(q, k, v, cta_k=oa.GPU_CTA_K, sm_scale=2 * 128 ** -0.5))
    wrong = wrong.astype(np.float64)
    assert (wrong * exact).sum() / np.sqrt((wrong * wrong).sum() * (exact * exact).sum()) < 0.99


def test_row_linear_rotation_cancels_against_rotated_weights():
    rng = np.random.default_rng(21)
    x = rng.standard_normal((16, 512)).astype(np.float32)
    x[:, rng.choice(512, 4, replace=False)] *= 20.0          # outlier channels, which ConvRot spreads
    w = (rng.standard_normal((96, 512)) * 0.05).astype(np.float32)
    wq, ws = o.quantize_rows(o.convrot256(w))                 # the checkpoint stores rotated weight rows
    exact = x.astype(np.float64) @ w.T.astype(np.float64)
    y = o.row_linear(x, wq, ws, out_dtype='f32', x_dtype='f32').astype(np.float64)
    rel = np.abs(y - exact).max() / np.abs(exact).max()
    assert rel < 0.02, rel
    # the same weights without the activation rotation are far off
    q, a = o.quantize_rows(x)
    plain = o.dequantize_row(o.int_mm(q, wq), a, ws, 'f32').astype(np.float64)
    assert np.abs(plain - exact).max() / np.abs(exact).max() > 0.2
    # the residual and gated forms cast the branch to FP16 first
    res = (rng.standard_normal((16, 96)) * 0.1).astype(np.float16)
    gate = rng.standard_normal((3, 96)).astype(np.float32)
    labels = np.arange(16) % 3
    x16 = x.astype(np.float16)
    branch = o.row_linear(x16, wq, ws, out_dtype='f16')
    assert np.array_equal(o.row_linear(x16, wq, ws, residual=res), o.residual_add(res, branch))
    assert np.array_equal(o.row_linear(x16, wq, ws, residual=res, gate=gate, labels=labels),
                          o.gated_residual_add(res, branch, gate, labels))


def test_rank_partials_sum_to_the_unsharded_accumulator():
    """Two rank halves of a row projection (whole 256-channel groups each):
    the MAX of the ranks' row maxima is the unsharded row maximum, and the
    int32 partials quantized with it add up to the unsharded accumulator."""
    rng = np.random.default_rng(17)
    m, k, n = 9, 1024, 48
    wq = rng.integers(-128, 128, (n, k), dtype=np.int8)
    # O projection: the K slice [0, k/2) on rank 0, [k/2, k) on rank 1
    x = (rng.standard_normal((m, k)) * 3).astype(np.float16)
    x[2] = 0
    halves = [x[:, :k // 2], x[:, k // 2:]]
    maxima = [o.rank_row_max(h) for h in halves]
    gmax = np.maximum(*maxima)
    assert np.array_equal(gmax, o.rank_row_max(x))
    assert not np.array_equal(maxima[0], gmax)      # the local maxima differ from the global
    parts = [o.row_partial(h, wq[:, r * k // 2:(r + 1) * k // 2], row_max=gmax) for r, h in enumerate(halves)]
    whole_acc, whole_a = o.row_partial(x, wq)
    assert np.array_equal(parts[0][0].astype(np.int64) + parts[1][0], whole_acc)
    assert np.array_equal(parts[0][1], whole_a) and np.array_equal(parts[1][1], whole_a)
    # a rank quantizing with its own maximum is a different operator
    own = o.row_partial(halves[0], wq[:, :k // 2])
    assert not np.array_equal(own[1], whole_a)
    # FC2: rank r holds [gate_r | up_r]; the unsharded input is [gate | up]
    w = 512
    gu = (rng.standard_normal((m, 2 * w)) * 2).astype(np.float16)
    gate, up = gu[:, :w], gu[:, w:]
    ranks = [np.concatenate([gate[:, r * w // 2:(r + 1) * w // 2], up[:, r * w // 2:(r + 1) * w // 2]], 1)
             for r in (0, 1)]
    wq2 = rng.integers(-128, 128, (n, w), dtype=np.int8)
    gmax2 = np.maximum(*[o.rank_row_max(r_, swiglu=True) for r_ in ranks])
    assert np.array_equal(gmax2, o.rank_row_max(gu, swiglu=True))
    p2 = [o.row_partial(r_, wq2[:, r * w // 2:(r + 1) * w // 2], row_max=gmax2, swiglu=True)
          for r, r_ in enumerate(ranks)]
    acc2, a2 = o.row_partial(gu, wq2, swiglu=True)
    assert np.array_equal(p2[0][0].astype(np.int64) + p2[1][0], acc2) and np.array_equal(p2[1][1], a2)
    # pairing rank 0's gate with rank 1's up breaks the identity
    swapped = np.concatenate([ranks[0][:, :w // 2], ranks[1][:, w // 2:]], 1)
    bad = o.row_partial(swapped, wq2[:, :w // 2], row_max=gmax2, swiglu=True)[0]
    assert not np.array_equal(bad.astype(np.int64) + p2[1][0], acc2)


# ------------------------------------------------ the reference attention kernel
def _qkv_np(rng, nq, nk, kshift=0.5):
    q = rng.standard_normal((1, 1, nq, 128)).astype(np.float16).astype(np.float32)
    k = (rng.standard_normal((1, 1, nk, 128)) + kshift).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((1, 1, nk, 128)).astype(np.float16).astype(np.float32)
    return q, k, v


def test_kitchen_restatement_pins():
    from oracle import int8_attention as oa
    assert abs(float(oa.S_U8_OFFSET) - np.log2(255.0)) < 1e-6     # exp2 of the offset is 255
    rng = np.random.default_rng(23)
    # identical keys: every non-last tile's probabilities are exactly 255, so
    # the output is the dequantized mean of V (the last tile sums its FP32
    # probabilities, 254.9999..., into the denominator: within 1e-6). The
    # centred identical keys have scales near the 1e-7 floor, which still
    # lets the -1e30 out-of-bounds score mask the padded keys of a partial
    # last block.
    for nk in (256, 250):
        q, _, v = _qkv_np(rng, 40, nk)
        k = np.repeat(rng.standard_normal((1, 1, 1, 128)).astype(np.float32), nk, axis=2)
        prep = oa.kitchen_prepare(q, k, v)
        assert np.all(prep['ksg'] < np.float32(2e-7))    # centred keys within fp32 rounding of zero
        out = oa.kitchen_attention(prep)
        want = (prep['v8'][0, 0, :nk].astype(np.float64).mean(0) * prep['vs'][0, 0])[None, :]
        assert np.abs(out[0, 0] - want).max() <= 1e-5 * np.abs(want).max(), nk
    # one key far above the rest: the output is that key's dequantized value row
    q, k, v = _qkv_np(rng, 8, 300)
    k[0, 0, 137] = q[0, 0, 0] * 40
    out = oa.kitchen_attention(oa.kitchen_prepare(q[:, :, :1], k, v))
    prep = oa.kitchen_prepare(q[:, :, :1], k, v)
    row = prep['v8'][0, 0, 137].astype(np.float64) * prep['vs'][0, 0]
    assert np.abs(out[0, 0, 0] - row).max() <= 1e-3 * np.abs(row).max()
    # the scales follow the kernel's thread grouping: rows 32 G + 8 i + j share
    # a Q scale, keys with the same (key mod 8) // 2 of a block share a K scale
    q, k, v = _qkv_np(rng, 70, 130)
    prep = oa.kitchen_prepare(q, k, v)
    qs, ks = prep['qs'][0, 0], prep['ks'][0, 0]
    assert qs[3] == qs[11] == qs[19] == qs[27] and qs[3] != qs[4]
    assert ks[2] == ks[3] == ks[10] == ks[11] and ks[2] != ks[4] and ks[2] != ks[66]


def test_kitchen_restatement_against_exact():
    """The restated reference scheme against exact float64 softmax attention
    (max-abs error over max |exact|), for both CTA_K choices of the reference
    launcher. The tile-relative u8 probabilities keep the error flat as the
    key count grows (a scheme quantizing P against the row maximum measured
    0.026 / 0.030 / 0.035 at 1000 / 4000 / 16384 keys)."""
    from oracle import int8_attention as oa
    rng = np.random.default_rng(29)
    for nq, nk, tol in ((64, 64, 0.02), (64, 1000, 0.02), (32, 4000, 0.02)):
        q, k, v = _qkv_np(rng, nq, nk)
        exact = oa.reference_attention(q, k, v)
        scale = np.abs(exact).max()
        for cta_k in (64, 128):
            ref = oa.kitchen_attention(oa.kitchen_prepare(q, k, v, cta_k=cta_k))
            assert np.abs(ref - exact).max() <= tol * scale, (nk, cta_k)
            cos = (ref * exact).sum() / np.sqrt((ref * ref).sum() * (exact * exact).sum())
            assert cos > 0.9998, (nk, cta_k, cos)
