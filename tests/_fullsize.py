"""Input builders and per-block oracle of the full-size parity tests (configs 2-4).

With causal attention the output rows of query block m of sequence z depend
only on that block's Q rows (their BLKQ quantisation block), the keys up to the
block's last row (their BLKK quantisation blocks, counted from the sequence's
first key) and routing row hk * ceil(Lq / 128) + m, so the oracle evaluated on
exactly that sub-problem reproduces those rows of a full-size launch.
"""
from __future__ import annotations

import numpy as np

from oracle import tilemix_oracle as O
from tilemix_amd.attention import precision_maps as pm

BM = 128
CFG2_OUTLIERS = (7, 33, 70, 101)


def _inputs(lengths, hq, hk, d, seed, head_scale=False, outliers=()):
    rng = np.random.default_rng(seed)
    n = int(sum(lengths))
    q = rng.standard_normal((n, hq, d), dtype=np.float32)
    k = rng.standard_normal((n, hk, d), dtype=np.float32)
    v = rng.standard_normal((n, hk, d), dtype=np.float32)
    if head_scale:  # per-head scale ~ U(0.5, 2)
        q *= rng.uniform(0.5, 2.0, size=(1, hq, 1)).astype(np.float32)
        k *= rng.uniform(0.5, 2.0, size=(1, hk, 1)).astype(np.float32)
        v *= rng.uniform(0.5, 2.0, size=(1, hk, 1)).astype(np.float32)
    for c in outliers:
        q[:, :, c] *= 8.0
        k[:, :, c] *= 8.0
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    return q.astype(np.float16), k.astype(np.float16), v.astype(np.float16), cu


def _oracle_block(q, k, v, cu, bits, hk, z, m, bnm, fp16_accum="exact"):
    """Oracle output of query block m of sequence z (Lq == Lk per sequence)."""
    s0, L = int(cu[z]), int(cu[z + 1] - cu[z])
    rows = min(BM, L - m * BM)
    kend = m * BM + rows
    qs = q[s0 + m * BM:s0 + m * BM + rows]
    ks, vs = k[s0:s0 + kend], v[s0:s0 + kend]
    cuq = np.array([0, rows], dtype=np.int32)
    cuk = np.array([0, kend], dtype=np.int32)
    mbz = -(-L // BM)
    sub_bits = np.array([int(bits[h * mbz + m]) for h in range(hk)], dtype=np.uint64)
    q8, sq, cuqs = O.quant_per_block_int8(qs, cuq, 128)
    k8, sk, cuks = O.quant_per_block_int8(ks, cuk, 64)
    return O.attn_fwd(qs, ks, vs, cuq, cuk, sub_bits, block_m=BM, block_n_mask=bnm, causal=True,
                      routing_mode=O.ROUTING_MIXED, q8=q8, k8=k8, sq16=sq.astype(np.float16),
                      sk16=sk.astype(np.float16), cu_q_scale=cuqs, cu_k_scale=cuks, fp16_accum=fp16_accum)


def _row_map(L, bnm, pattern, params, hk):
    row = pm.make_precision_bitmask(L, BM, bnm, None, percentage=0.5, pattern_type=pattern,
                                    pattern_params=params, COMPUTE_BLOCK_N=64)
    return np.array([int(x) for x in row.tolist()] * hk, dtype=np.uint64)


# cfg2 query blocks checked: first, middle and the last (4096-key) blocks
CFG2_BLOCKS = ((0, 0), (0, 17), (3, 17), (3, 31), (7, 31))
# Bound on the max-abs distance to the exact-sum oracle at cfg2 (see
# test_cfg2_full_size_blocks in test_gpu_fullsize.py); the CPU comparison of
# accumulation models (test_accumulation_models.py) measures up to 2.4e-2 for
# fp32 accumulation alone on these inputs.
CFG2_EXACT_MAX_ABS = 5e-2
