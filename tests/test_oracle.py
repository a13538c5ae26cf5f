"""Pin the CPU oracle (oracle/tilemix_oracle.py) before trusting it as the checker.

The reference ships no tests and no golden vectors (the routing-map fixtures
of test_precision_maps.py were written by this repository's
tests/golden/make_precision_map_goldens.py from the reference's own module), so
every oracle function is checked here against something that does not restate
its formula:

* quantisation: closed-form invariants, exact half-way rounding cases, and an
  element-by-element scalar restatement on small blocks;
* int32 Q8.K8 accumulators: a textbook integer GEMM in int64;
* attention at an all-FP16 map: fp64 softmax(QK^T)V within fp16 rounding,
  including Lq != Lk (causal offset), GQA and varlen packing;
* INT8 route: fp64 attention over the dequantised scores;
* one 64-key tile: brute force of the online-softmax update;
* routing rows / bits: per-element bit extraction.

A mutation harness then re-executes the oracle's own source with one planted
mistake at a time (wrong causal offset, dropped 1/l, wrong GQA head map,
wrong route bit, round-half-even instead of half-away, missing softmax scale
in the INT8 dequant, inverted alpha) and requires every mutant to fail at
least one of the checks above.  Everything runs on the CPU.
"""
from __future__ import annotations

import types

import numpy as np
import pytest

from oracle import tilemix_oracle as O

f16, f32 = np.float16, np.float32


# ----------------------------------------------------------------- helpers
def _inputs(lengths, hq, hk, d, seed, scale=1.0, lq=None):
    rng = np.random.default_rng(seed)
    nk = int(sum(lengths))
    lq = lengths if lq is None else lq
    nq = int(sum(lq))
    q = (rng.standard_normal((nq, hq, d)) * scale).astype(f16)
    k = (rng.standard_normal((nk, hk, d)) * scale).astype(f16)
    v = rng.standard_normal((nk, hk, d)).astype(f16)
    cu_k = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    cu_q = np.concatenate([[0], np.cumsum(lq)]).astype(np.int64)
    return q, k, v, cu_q, cu_k


def _fp64_attention(q, k, v, cu_q, cu_k, causal, sm_scale=None, scores=None):
    """softmax(q k^T * sm_scale) v in float64 (or of given per-(z,h) scores)."""
    nq, hq, d = q.shape
    group = hq // k.shape[1]
    sm = d ** -0.5 if sm_scale is None else sm_scale
    out = np.zeros((nq, hq, d))
    for z in range(len(cu_q) - 1):
        qs, lq = cu_q[z], cu_q[z + 1] - cu_q[z]
        ks, lk = cu_k[z], cu_k[z + 1] - cu_k[z]
        if lq == 0:
            continue
        for h in range(hq):
            hk = h // group
            if scores is None:
                s = q[qs:qs + lq, h].astype(np.float64) @ k[ks:ks + lk, hk].astype(np.float64).T * sm
            else:
                s = scores(z, h)
            if causal:
                mask = np.arange(lk)[None, :] <= np.arange(lq)[:, None] + (lk - lq)
                s = np.where(mask, s, -np.inf)
            mx = s.max(axis=1, keepdims=True)
            mx = np.where(np.isfinite(mx), mx, 0.0)
            p = np.exp(s - mx)
            den = p.sum(axis=1, keepdims=True)
            den = np.where(den > 0, den, 1.0)
            out[qs:qs + lq, h] = (p / den) @ v[ks:ks + lk, hk].astype(np.float64)
    return out


def _all_bits(hk, m_blocks, value):
    return np.full(hk * m_blocks, np.uint64(value), dtype=np.uint64)


# ---------------------------------------------------------------- checks
# Each check takes the oracle module (real or mutant) and raises AssertionError
# on a mismatch.

def check_quant_invariants(Om):
    rng = np.random.default_rng(1)
    lengths = [1, 63, 64, 65, 200]
    x = rng.standard_normal((sum(lengths), 3, 32)).astype(np.float32)
    x[:, :, 5] *= 30.0
    x = x.astype(f16)
    cu = np.concatenate([[0], np.cumsum(lengths)])
    for blk in (64, 128):
        codes, scale, cus = Om.quant_per_block_int8(x, cu, blk)
        assert cus.tolist() == np.concatenate([[0], np.cumsum([(L + blk - 1) // blk for L in lengths])]).tolist()
        assert codes.min() >= -127 and codes.max() <= 127
        for b, L in enumerate(lengths):
            for j in range((L + blk - 1) // blk):
                t0, t1 = cu[b] + j * blk, cu[b] + min((j + 1) * blk, L)
                blkx = x[t0:t1].astype(np.float64)
                for h in range(3):
                    s = np.float64(scale[cus[b] + j, h])
                    amax = np.abs(blkx[:, h]).max()
                    assert s == np.float64(f32(f32(amax) / f32(127.0)))
                    c = codes[t0:t1, h].astype(np.float64)
                    # the element of largest magnitude maps to +-127
                    i = np.unravel_index(np.abs(blkx[:, h]).argmax(), blkx[:, h].shape)
                    assert abs(c[i]) == 127
                    # round-half-away reconstruction bound
                    assert np.all(np.abs(blkx[:, h] - c * s) <= s * 0.5 * (1 + 1e-5) + 1e-30)


def check_quant_halfway(Om):
    # amax = 127 -> scale exactly 1.0: x / s = x, so x = k + 0.5 is an exact tie.
    vals = np.array([127.0, 2.5, -2.5, 0.5, -0.5, 1.5, 3.5, -0.25, 0.0], dtype=f16)
    x = np.zeros((64, 1, 16), dtype=f16)
    x[:len(vals), 0, 0] = vals
    codes, scale, _ = Om.quant_per_block_int8(x, [0, 64], 64)
    assert scale[0, 0] == f32(1.0)
    assert codes[:len(vals), 0, 0].tolist() == [127, 3, -3, 1, -1, 2, 4, 0, 0]


def check_quant_bruteforce(Om):
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((40, 2, 8)) * rng.uniform(0.01, 50)).astype(f16)
    for sm in (1.0, 0.0883883):
        codes, scale, _ = Om.quant_per_block_int8(x, [0, 40], 64, sm_scale=sm)
        for h in range(2):
            ref, s = O.quant_block_scalar(x[:, h], sm_scale=sm)
            assert scale[0, h] == s
            assert codes[:, h].reshape(-1).tolist() == ref.tolist()


def check_quant_zero_and_tail(Om):
    x = np.zeros((70, 1, 16), dtype=f16)
    x[64:, 0, :] = np.arange(6 * 16, dtype=np.float32).reshape(6, 16).astype(f16)
    codes, scale, cus = Om.quant_per_block_int8(x, [0, 70], 64)
    assert cus.tolist() == [0, 2]
    assert scale[0, 0] == 0 and (codes[:64] == 0).all()          # all-zero block: scale 0, codes 0
    assert scale[1, 0] == f32(f32(95.0) / f32(127.0))             # tail block: 6 rows only
    assert codes[69, 0, 15] == 127


def check_int32_accumulators(Om):
    q, k, v, cu_q, cu_k = _inputs([80, 130], 4, 2, 64, seed=3)
    q8, sq, cuq = Om.quant_per_block_int8(q, cu_q, 128)
    k8, sk, cuk = Om.quant_per_block_int8(k, cu_k, 64)
    mb = (130 + 63) // 64
    _, scores = Om.attn_fwd(q, k, v, cu_q, cu_k, _all_bits(2, mb, ~np.uint64(0)), block_m=64, block_n_mask=64,
                            causal=True, routing_mode=O.ROUTING_INT8, q8=q8, k8=k8, sq16=sq.astype(f16),
                            sk16=sk.astype(f16), cu_q_scale=cuq, cu_k_scale=cuk, want_scores=True)
    for z in range(2):
        for h in range(4):
            acc, _, _ = scores[(z, h)]
            qa = q8[cu_q[z]:cu_q[z + 1], h].astype(np.int64)
            ka = k8[cu_k[z]:cu_k[z + 1], h // 2].astype(np.int64)
            exact = np.einsum("qd,kd->qk", qa, ka)
            assert np.array_equal(acc, exact)


FP16_CASES = [
    # lengths (keys), lq (queries) or None, hq, hk, d, causal
    ([64], None, 2, 1, 64, True),
    ([200, 37, 128], None, 4, 2, 64, True),
    ([190], [150], 3, 1, 32, True),      # Lq != Lk: causal offset Lk - Lq
    ([96, 160], None, 4, 4, 32, False),
]


def check_fp16_attention(Om):
    for lengths, lq, hq, hk, d, causal in FP16_CASES:
        q, k, v, cu_q, cu_k = _inputs(lengths, hq, hk, d, seed=len(lengths) + d, lq=lq)
        lmax = max(int(x) for x in np.diff(cu_q))
        mb = (lmax + 63) // 64
        out = Om.attn_fwd(q, k, v, cu_q, cu_k, _all_bits(hk, mb, 0), block_m=64, block_n_mask=64, causal=causal)
        ref = _fp64_attention(q, k, v, cu_q, cu_k, causal)
        err = np.abs(out.astype(np.float64) - ref)
        assert err.max() < 4e-3 and err.mean() < 4e-4, (lengths, err.max(), err.mean())


def check_int8_attention(Om):
    q, k, v, cu_q, cu_k = _inputs([150, 70], 4, 2, 64, seed=11)
    q8, sq, cuq = Om.quant_per_block_int8(q, cu_q, 128)
    k8, sk, cuk = Om.quant_per_block_int8(k, cu_k, 64)
    sq16, sk16 = sq.astype(f16), sk.astype(f16)
    out = Om.attn_fwd(q, k, v, cu_q, cu_k, _all_bits(2, 3, ~np.uint64(0)), block_m=64, block_n_mask=64,
                      causal=True, routing_mode=O.ROUTING_INT8, q8=q8, k8=k8, sq16=sq16, sk16=sk16,
                      cu_q_scale=cuq, cu_k_scale=cuk)

    def scores(z, h):
        qa = q8[cu_q[z]:cu_q[z + 1], h].astype(np.float64)
        ka = k8[cu_k[z]:cu_k[z + 1], h // 2].astype(np.float64)
        lq, lk = qa.shape[0], ka.shape[0]
        rq = sq16[cuq[z] + np.arange(lq) // 128, h].astype(np.float64)
        rk = sk16[cuk[z] + np.arange(lk) // 64, h // 2].astype(np.float64)
        return (qa @ ka.T) * rq[:, None] * rk[None, :] * 64 ** -0.5

    ref = _fp64_attention(q, k, v, cu_q, cu_k, True, scores=scores)
    err = np.abs(out.astype(np.float64) - ref)
    assert err.max() < 4e-3 and err.mean() < 4e-4, (err.max(), err.mean())


def _single_tile(Om, L, block_n):
    # One tile: m = row max, alpha = 0 on the first tile, l = sum fp16(p).
    q, k, v, cu_q, cu_k = _inputs([L], 1, 1, 32, seed=5, scale=2.0)
    out = Om.attn_fwd(q, k, v, cu_q, cu_k, _all_bits(1, -(-L // 64), 0), block_m=64, block_n_mask=256,
                      causal=True, block_n=block_n)
    qk_scale = f32(f32(32 ** -0.5) * f32(O.LOG2E))
    q16 = (q[:, 0].astype(f32) * qk_scale).astype(f16)
    for r in range(0, L, max(1, L // 48)):
        s = [f16(np.dot(q16[r].astype(np.float64), k[j, 0].astype(np.float64))) for j in range(r + 1)]
        m = max(float(x) for x in s)
        p = [f16(np.exp2(f32(f32(x) - f32(m)))) for x in s]
        den = sum(float(x) for x in p)
        num = sum(float(p[j]) * v[j, 0].astype(np.float64) for j in range(r + 1))
        ref = num / den
        assert np.abs(out[r, 0].astype(np.float64) - ref).max() <= 2.0 ** -10 * max(1.0, np.abs(ref).max())


def check_single_tile(Om):
    _single_tile(Om, 48, 64)


def check_single_tile_block_n256(Om):
    # 200 keys are one softmax step at block_n = 256.
    _single_tile(Om, 200, 256)


def check_block_n_known_answer(Om):
    """One row of 65 keys with given fp16 scores 0 (keys 0-63) and 0.5 (key 64),
    V = 1 on keys 0-63 and -45 on key 64.  block_n >= 128 is one softmax step:
    m = 0.5 before any p, p = fp16(2^-0.5) on keys 0-63, so
    out = (64 p - 45) / (64 p + 1).  block_n = 64 takes p = 1 under m = 0 and
    then rescales by alpha = fp32(2^-0.5): out = (64 alpha - 45) / (64 alpha + 1).
    The two differ by ~1e-4 (~27 fp16 ulps of the output)."""
    L = 65
    q = np.zeros((L, 1, 16), f16)
    k = np.zeros((L, 1, 16), f16)
    v = np.zeros((L, 1, 16), f16)
    v[:64, 0, 0] = 1
    v[64, 0, 0] = -45
    s = np.zeros((L, L), f16)
    s[:, 64] = 0.5
    cu = np.array([0, L])
    got = {}
    for bn in (64, 128, 256):
        out = Om.attn_fwd(q, k, v, cu, cu, _all_bits(1, 2, 0), block_m=64, block_n_mask=256, causal=False,
                          qk16_override=lambda z, h: s, block_n=bn)
        assert (out[:, 0, 0] == out[0, 0, 0]).all()
        got[bn] = out[0, 0, 0]
    p = f32(f16(np.exp2(f32(-0.5))))
    alpha = f32(np.exp2(f32(-0.5)))
    want_one_step = f16(f32(f32(64) * p - f32(45)) / f32(f32(64) * p + f32(1)))
    want_two_steps = f16(f32(f32(64) * alpha - f32(45)) / f32(f32(64) * alpha + f32(1)))
    assert want_one_step != want_two_steps
    assert got[128] == want_one_step and got[256] == want_one_step, (got, want_one_step)
    assert got[64] == want_two_steps, (got, want_two_steps)


def check_block_n_fp16_attention(Om):
    # block_n 128 / 256 against fp64 softmax attention (varlen, causal, GQA).
    q, k, v, cu_q, cu_k = _inputs([300, 129, 1], 4, 2, 64, seed=12)
    for bn in (128, 256):
        out = Om.attn_fwd(q, k, v, cu_q, cu_k, _all_bits(2, 5, 0), block_m=64, block_n_mask=256, causal=True,
                          block_n=bn)
        ref = _fp64_attention(q, k, v, cu_q, cu_k, True)
        err = np.abs(out.astype(np.float64) - ref)
        assert err.max() < 4e-3 and err.mean() < 4e-4, (bn, err.max(), err.mean())


def check_int8_vector_scales(Om):
    """INT8 route with K scale blocks of 16, 32 and 48 keys (the per-key lookup
    sk[key // BLKK], reference :390) and block_n 128: fp64 attention over the
    dequantised scores."""
    q, k, v, cu_q, cu_k = _inputs([150, 70], 4, 2, 64, seed=13)
    q8, sq, cuq = Om.quant_per_block_int8(q, cu_q, 128)
    sq16 = sq.astype(f16)
    for blkk, bn in ((16, 64), (32, 128), (48, 64)):
        k8, sk, cuk = Om.quant_per_block_int8(k, cu_k, blkk)
        sk16 = sk.astype(f16)
        out = Om.attn_fwd(q, k, v, cu_q, cu_k, _all_bits(2, 3, ~np.uint64(0)), block_m=64, block_n_mask=128,
                          causal=True, routing_mode=O.ROUTING_INT8, q8=q8, k8=k8, sq16=sq16, sk16=sk16,
                          cu_q_scale=cuq, cu_k_scale=cuk, blkk=blkk, block_n=bn)

        def scores(z, h):
            qa = q8[cu_q[z]:cu_q[z + 1], h].astype(np.float64)
            ka = k8[cu_k[z]:cu_k[z + 1], h // 2].astype(np.float64)
            lq, lk = qa.shape[0], ka.shape[0]
            rq = sq16[cuq[z] + np.arange(lq) // 128, h].astype(np.float64)
            rk = sk16[cuk[z] + np.arange(lk) // blkk, h // 2].astype(np.float64)
            return (qa @ ka.T) * rq[:, None] * rk[None, :] * 64 ** -0.5

        ref = _fp64_attention(q, k, v, cu_q, cu_k, True, scores=scores)
        err = np.abs(out.astype(np.float64) - ref)
        assert err.max() < 4e-3 and err.mean() < 4e-4, (blkk, err.max(), err.mean())


def check_route_table(Om):
    rng = np.random.default_rng(2)
    bm = rng.integers(0, 2 ** 63, size=3 * 4, dtype=np.uint64) * np.uint64(2) + np.uint64(1)
    for bnm in (64, 128, 256):
        t = Om.route_table(bm, hk=2, Lq=220, Lk=500, block_m=64, block_n_mask=bnm, routing_mode=O.ROUTING_MIXED)
        mbz, nt = 4, 8
        assert t.shape == (mbz, nt)
        for m in range(mbz):
            for n in range(nt):
                assert t[m, n] == bool((int(bm[2 * mbz + m]) >> (n * 64 // bnm)) & 1)


CHECKS = [check_quant_invariants, check_quant_halfway, check_quant_bruteforce, check_quant_zero_and_tail,
          check_int32_accumulators, check_fp16_attention, check_int8_attention, check_single_tile,
          check_single_tile_block_n256, check_block_n_known_answer, check_block_n_fp16_attention,
          check_int8_vector_scales, check_route_table]


@pytest.mark.parametrize("check", CHECKS, ids=[c.__name__ for c in CHECKS])
def test_oracle_pinned(check):
    check(O)


# ------------------------------------------------------------- mutations
MUTATIONS = {
    "causal_offset": ("keys[None, :] <= rows[:, None] + (Lk - Lq)", "keys[None, :] <= rows[:, None]"),
    "dropped_inv_l": ("(acc / l_i[:, None]).astype(f16)", "(acc).astype(f16)"),
    "gqa_head_map": ("hk = h // group", "hk = h % hkv"),
    "route_bit": ("shifts = (np.arange(nt) // group)", "shifts = (np.arange(nt))"),
    "round_half_even": ("t = (t + np.where(t >= 0, f32(0.5), f32(-0.5))).astype(f32)", "t = np.rint(t).astype(f32)"),
    "dequant_no_qk_scale": ("ss = (sqk.astype(f32) * qk_scale).astype(f16)",
                            "ss = (sqk.astype(f32) * f32(O_LOG2E_ONLY)).astype(f16)"),
    "inverted_alpha": ("np.exp2(m_i - m_next)", "np.exp2(m_next - m_i)"),
    # softmax steps of 64 keys whatever block_n is (every key still visited)
    "softmax_step_64": [("nt = _ceil_div(Lk, block_n)", "nt = _ceil_div(Lk, BN)"),
                        ("k0, k1 = n * block_n, min((n + 1) * block_n, Lk)", "k0, k1 = n * BN, min((n + 1) * BN, Lk)")],
    "k_scale_block_64": ("int(cu_k_scale[z + 1]),\n                                 keys // blkk",
                         "int(cu_k_scale[z + 1]),\n                                 keys // 64"),
}


def _mutant(name):
    src = open(O.__file__).read()
    pairs = MUTATIONS[name]
    for old, new in ([pairs] if isinstance(pairs, tuple) else pairs):
        assert src.count(old) == 1, f"mutation anchor for {name} not unique"
        src = src.replace(old, new)
    mod = types.ModuleType(f"oracle_mutant_{name}")
    mod.__dict__["O_LOG2E_ONLY"] = O.LOG2E
    exec(compile(src, f"<mutant {name}>", "exec"), mod.__dict__)
    return mod


@pytest.mark.parametrize("name", sorted(MUTATIONS))
def test_planted_mistake_is_caught(name):
    mod = _mutant(name)
    failures = []
    for check in CHECKS:
        try:
            check(mod)
        except AssertionError:
            failures.append(check.__name__)
    assert failures, f"mutation {name} passed every oracle check"
