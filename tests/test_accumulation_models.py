"""FP16-route score accumulation: the models of oracle.fp16_tile_scores, pinned,
and what the accumulation order alone does to cfg2's outputs (CPU only, no kernel).

The reference's FP16 tile computes ``tl.dot(q16, k, out_dtype=float16)``
(attention/triton/tilemix.py:254): how that sum accumulates belongs to Triton
and the GPU (unpinned).  The oracle's definition is the exact sum rounded once
to fp16; the gfx950 kernel accumulates in fp32, one 16-wide k-step per MFMA
(modelled by ``fp32_k16``; the instruction's internal summation is not exactly
that model's, but its fp16 scores equal the exact sum's on >= 99.9% of entries,
GPU test test_cfg2_decomposed_strict).  On cfg2's inputs (4 channels
x8 in Q and K) the softmax is peaked enough that the one-ulp score moves of fp32
accumulation move an output by up to ~2e-2 -- measured here between two CPU
oracles, so the spread is a property of fp32 accumulation, not of the kernel.
An fp16 accumulator (``fp16_k16``, a model of an fp16-accumulating dot) moves
outputs far more, past the mean-abs bar.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import tilemix_oracle as O
from tests._fullsize import CFG2_EXACT_MAX_ABS, CFG2_OUTLIERS, _inputs, _oracle_block, _row_map

f16, f32 = np.float16, np.float32


def test_models_agree_when_every_partial_sum_is_exact():
    """Small integers: every partial sum is representable in fp16, so all three
    models give the exact dot product."""
    rng = np.random.default_rng(0)
    q = rng.integers(-3, 4, size=(5, 64)).astype(f16)
    k = rng.integers(-3, 4, size=(7, 64)).astype(f16)
    exact = (q.astype(np.int64) @ k.astype(np.int64).T).astype(f16)
    for accum in ("exact", "fp32_k16", "fp16_k16"):
        np.testing.assert_array_equal(O.fp16_tile_scores(q, k, accum), exact)


def test_known_answer_where_fp16_accumulation_loses_bits():
    """q = (2048, 1, 0.., 1 in each later 16-slice), k = ones: the exact dot is
    2048 + 8 = 2056.  An fp16 accumulator at 2048 (ulp 2) drops every +1 (a tie,
    rounded to even), giving 2048; fp32 keeps them."""
    q = np.zeros((1, 128), dtype=f16)
    q[0, 0] = 2048
    q[0, 1] = 1
    for s in range(1, 8):
        q[0, 16 * s] = 1
    k = np.ones((1, 128), dtype=f16)
    assert float(O.fp16_tile_scores(q, k, "exact")[0, 0]) == 2056.0
    assert float(O.fp16_tile_scores(q, k, "fp32_k16")[0, 0]) == 2056.0
    assert float(O.fp16_tile_scores(q, k, "fp16_k16")[0, 0]) == 2048.0


def test_fp32_k16_against_scalar_loop():
    """k16_accumulate against a plain scalar loop (Python floats for the exact
    slice sums, numpy fp32 for each rounding) on random fp16 data."""
    rng = np.random.default_rng(1)
    q = (rng.standard_normal((3, 64)) * 4).astype(f16)
    k = (rng.standard_normal((4, 64)) * 4).astype(f16)
    got = O.k16_accumulate(q, k, f32)
    for i in range(3):
        for j in range(4):
            acc = f32(0.0)
            for s in range(4):
                part = 0.0
                for d in range(16 * s, 16 * s + 16):
                    part += float(q[i, d]) * float(k[j, d])  # exact: few terms, small exponent range
                acc = f32(float(acc) + part)
            assert got[i, j] == acc


def test_cfg2_spread_of_accumulation_order():
    """cfg2's inputs, the query blocks of the GPU test: the fp32-k16 oracle vs
    the exact oracle.  Mean-abs stays far under 2e-4, max-abs exceeds 2e-3 on
    some block (one-ulp score moves in a peaked softmax) and stays within the
    bound the GPU test holds the kernel to; the fp16-k16 model fails the
    mean-abs bar."""
    lengths, hq, hk = [4096] * 8, 24, 8
    q, k, v, cu = _inputs(lengths, hq, hk, 128, seed=2, outliers=CFG2_OUTLIERS)
    bits = _row_map(4096, 64, "sptrans", {"stride": 128, "c": 32}, hk)
    worst32 = 0.0
    for z, m in ((0, 31), (3, 17)):
        ref = _oracle_block(q, k, v, cu, bits, hk, z, m, 64).astype(np.float64)
        o32 = _oracle_block(q, k, v, cu, bits, hk, z, m, 64, fp16_accum="fp32_k16").astype(np.float64)
        o16 = _oracle_block(q, k, v, cu, bits, hk, z, m, 64, fp16_accum="fp16_k16").astype(np.float64)
        d32, d16 = np.abs(o32 - ref), np.abs(o16 - ref)
        print(f"block ({z},{m}): fp32_k16 vs exact max {d32.max():.3e} mean {d32.mean():.3e}; "
              f"fp16_k16 vs exact max {d16.max():.3e} mean {d16.mean():.3e}")
        assert d32.mean() <= 2e-5 and d32.max() <= CFG2_EXACT_MAX_ABS
        assert d16.mean() > 2e-4
        worst32 = max(worst32, d32.max())
    assert worst32 > 2e-3


@pytest.mark.parametrize("accum", ["fp32_k16", "fp16_k16"])
def test_planted_accumulation_error_is_caught(accum):
    """A model that dropped the last k-slice would not match the scalar loop."""
    rng = np.random.default_rng(2)
    q = rng.standard_normal((2, 32)).astype(f16)
    k = rng.standard_normal((3, 32)).astype(f16)
    full = O.k16_accumulate(q, k, f32 if accum == "fp32_k16" else f16)
    dropped = O.k16_accumulate(q[:, :16], k[:, :16], f32 if accum == "fp32_k16" else f16)
    assert not np.array_equal(full, dropped)
