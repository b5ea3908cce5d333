"""The FC2 prologue's SwiGLU division for fp16 gates, evaluated exactly on the CPU.

For a gate g in (-44, 2^16) the kernel (`swiglu_fp16_gate` in
csrc/w8a8_device.h) forms g / den, den = 1 + exp(-g), as
    r = hardware reciprocal of den (within 1 ulp of 1/den),
    q = fp32(g * r),
    a = fp32(q + fp32(g - den * q) * r)      (two single-rounding FMAs)
and claims a equals the IEEE quotient fp32(g / den) for every such gate. The
hardware reciprocal is not modelled bit for bit: r is taken as each fp32
neighbour of the exact 1/den (one of them is the correctly rounded value).
Every step is evaluated with integers, so no double rounding can hide a
mismatch. The GPU tests run every finite fp16 gate through the kernel itself.
"""
import math

import numpy as np

import oracle as o

F32 = np.float32


def _parts(x):
    """(m, e) with float x = m * 2**e exactly, m an int."""
    m, e = math.frexp(x)
    return int(m * (1 << 53)), e - 53


def _round_f32(m, e):
    """fp32 nearest to m * 2**e (ties to even); the values here are normal."""
    if m == 0:
        return 0.0
    sign = -1 if m < 0 else 1
    m = abs(m)
    drop = m.bit_length() - 24            # keep 24 significant bits
    if drop > 0:
        q, r = m >> drop, m & ((1 << drop) - 1)
        half = 1 << (drop - 1)
        if r > half or (r == half and q & 1):
            q += 1
        m, e = q, e + drop
    return sign * math.ldexp(m, e)


def _fma_f32(a, b, c):
    """fp32(a * b + c) with one rounding, for fp32 values a, b, c."""
    ma, ea = _parts(a)
    mb, eb = _parts(b)
    mc, ec = _parts(c)
    mp, ep = ma * mb, ea + eb
    e = min(ep, ec)
    return _round_f32((mp << (ep - e)) + (mc << (ec - e)), e)


def _kernel_division(g, den, r):
    q = _fma_f32(g, r, 0.0)
    return _fma_f32(_fma_f32(-den, q, g), r, q)


def _neighbours_of_reciprocal(den):
    rn = F32(1) / F32(den)                  # the correctly rounded reciprocal
    exact_above = float(rn) * den < 1.0     # is 1/den above rn?
    other = np.nextafter(rn, F32(np.inf) if exact_above else F32(0))
    return float(rn), float(other)


def test_reciprocal_division_equals_ieee_for_every_fp16_gate():
    bits = np.arange(65536, dtype=np.uint32)
    finite = bits[(bits & 0x7C00) != 0x7C00].astype(np.uint16).view(np.float16).astype(F32)
    g32 = finite[(finite > -44) & (finite < 65536) & (finite != 0)]
    den32 = (F32(1) + o.exp_f32(-g32)).astype(F32)
    want32 = (g32 / den32).astype(F32)
    assert g32.size == 52606
    needs_rn = []
    for g, den, want in zip(g32.tolist(), den32.tolist(), want32.tolist()):
        rn, other = _neighbours_of_reciprocal(den)
        assert _kernel_division(g, den, rn) == want, (g, den)
        if _kernel_division(g, den, other) != want:
            needs_rn.append(g)
    # One gate needs the correctly rounded reciprocal: g = 2^-23 with
    # den = 2 - 2^-23, whose quotient 2^-24 / (1 - 2^-24) lies 2^-48 above the
    # midpoint between 2^-24 and its successor.
    assert needs_rn == [2.0 ** -23]


def test_exact_fma_helper_against_hand_values():
    # 1 + 2^-24 is a tie between 1 and 1 + 2^-23: rounds to even (1.0); a
    # hair above rounds up.
    assert _fma_f32(1.0, 1.0, 2.0 ** -24) == 1.0
    assert _fma_f32(1.0 + 2.0 ** -23, 1.0, 2.0 ** -24) == 1.0 + 2.0 ** -22
    # Exact value 1 + 2^-24 + 2^-70, above the tie: float64 arithmetic rounds
    # it onto the tie first, and ties-to-even would then give 1.0.
    a, b, c = -(1.0 + 2.0 ** -23) * 2.0 ** -24, 1.0 - 2.0 ** -23, 1.0 + 2.0 ** -23
    assert float(F32(a * b + c)) == 1.0
    assert _fma_f32(a, b, c) == 1.0 + 2.0 ** -23
    assert _fma_f32(1.0 + 2.0 ** -23, 1.0 + 2.0 ** -23, -1.0) == float(F32(2.0 ** -22 + 2.0 ** -46))
    assert _fma_f32(3.0, 5.0, -15.0) == 0.0
