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
