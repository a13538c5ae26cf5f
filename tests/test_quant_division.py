"""The quantisation kernels divide by the block scale through an IEEE
reciprocal and one FMA correction step (``div_by_recip`` in
tilemix_amd/csrc/attn_common.h): q0 = RN(x r), rem = fma(-q0, s, x),
q1 = fma(rem, r, q0), r = RN(1 / s).  The reference divides (x / s).  This
test checks, on the CPU, that both give the same quotient -- and so the same
int8 code -- for every fp16 x with |x| <= amax, for amax spread over every
fp16 exponent (all mantissas at the extremes).  The two FMAs are emulated in
float64, where both are exact before the single rounding to float32: the
remainder is exactly representable and |rem r| is below one ulp of q0.

(The kernels' own GPU arithmetic was checked the same way on every positive
fp16 amax: 1.0e9 pairs, no difference in value or code.)
"""
from __future__ import annotations

import numpy as np

f32 = np.float32


def _fma32(a, b, c):
    return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(f32)


def _amax_samples():
    bits = set()
    for e in range(0, 31):                      # every fp16 exponent (0 = subnormal)
        base = e << 10
        for m in (0, 1, 2, 3, 0x155, 0x2AA, 0x3FD, 0x3FE, 0x3FF):
            bits.add(base | m)
        rng = np.random.default_rng(e)
        bits.update(int(x) for x in base | rng.integers(0, 1024, size=6))
    bits.discard(0)
    return np.array(sorted(bits), dtype=np.uint16).view(np.float16).astype(f32)


def test_reciprocal_division_equals_ieee_division():
    xs_all = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(f32)
    xs_all = xs_all[np.isfinite(xs_all)]
    checked = 0
    for amax in _amax_samples():
        x = xs_all[np.abs(xs_all) <= amax]
        s = f32(amax / f32(127.0))
        r = f32(f32(1.0) / s)
        with np.errstate(over="ignore"):
            t_div = (x / s).astype(f32)
            q0 = (x * r).astype(f32)
        rem = _fma32(-q0, np.full_like(x, s), x)
        q1 = _fma32(rem, np.full_like(x, r), q0)
        assert np.array_equal(q1, t_div), f"amax={amax}"      # -0 == +0
        code = lambda t: np.trunc(t + np.where(t >= 0, f32(0.5), f32(-0.5))).astype(np.int64)
        assert np.array_equal(code(q1), code(t_div)), f"amax={amax}"
        checked += x.size
    assert checked > 10_000_000


def _rn32_exact(x):
    """Round a Fraction to the nearest float32 (ties to even), normal range."""
    from fractions import Fraction
    if x == 0:
        return Fraction(0)
    sign = -1 if x < 0 else 1
    x = abs(x)
    e = x.numerator.bit_length() - x.denominator.bit_length()
    if Fraction(2) ** e > x:
        e -= 1
    if Fraction(2) ** (e + 1) <= x:
        e += 1
    scale = Fraction(2) ** (23 - e)
    m = x * scale
    q, r = divmod(m.numerator, m.denominator)
    if 2 * r > m.denominator or (2 * r == m.denominator and q & 1):
        q += 1
    return sign * Fraction(q) / scale


def test_reciprocal_division_epilogue_domain():
    """The attention epilogue computes acc / l the same way (r = RN(1/l), two
    FMAs).  There the remainder is not always representable, so each FMA is
    evaluated in exact rational arithmetic with one rounding to float32; on
    random (acc, l) over the kernel's range (l in [1, 8192], |acc| in
    [1e-6, 1e4]) the result equals the correctly rounded quotient."""
    from fractions import Fraction
    rng = np.random.default_rng(7)
    n = 20000
    ls = np.where(rng.random(n) < 0.3, rng.uniform(1.0, 2.0, n), rng.uniform(1.0, 8192.0, n)).astype(f32)
    accs = (rng.choice([-1.0, 1.0], n) * 10.0 ** rng.uniform(-6, 4, n)).astype(f32)
    inexact = 0
    for a32, l32 in zip(accs, ls):
        a, lv = Fraction(float(a32)), Fraction(float(l32))
        r = _rn32_exact(1 / lv)
        q0 = _rn32_exact(a * r)
        rem = _rn32_exact(a - q0 * lv)
        inexact += rem != a - q0 * lv
        q1 = _rn32_exact(q0 + rem * r)
        assert q1 == _rn32_exact(a / lv), (float(a32), float(l32))
    assert inexact > 0  # the sample reaches the cases where the first FMA rounds
