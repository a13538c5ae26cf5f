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
* INT8 route on int8 V codes: fp64 attention over the dequantised scores and
  the dequantised V (BLKK 64 and 16), and a hand-derived known answer in which
  the fp16 rounding of p * sv changes the output;
* bias: a hand-derived known answer in which LOG2E taken at fp16 changes a
  score, fp64 attention over scores plus bias, and the batch-0 reading of the
  bias in a two-sequence launch;
* one 64-key tile: brute force of the online-softmax update;
* routing rows / bits: per-element bit extraction.

A mutation harness then re-executes the oracle's own source with one planted
mistake at a time (wrong causal offset, dropped 1/l, wrong GQA head map,
wrong route bit, round-half-even instead of half-away, missing softmax scale
in the INT8 dequant, inverted alpha, softmax steps of 64 keys, K scale blocks
of 64, the V scale dropped, fp16 V on INT8 tiles, p * sv unrounded, the bias's
LOG2E dropped or taken in fp32, a per-sequence or transposed bias) and
requires every mutant to fail at least one of the checks above.  Everything
runs on the CPU.
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


def _int8_v_setup(seed, blkk):
    """INT8-route inputs with int8 V codes: V ~ 4 N(0,1), so one code step
    (~0.11) is far above the output tolerance."""
    q, k, v, cu_q, cu_k = _inputs([150, 70], 4, 2, 64, seed=seed)
    v = (v.astype(f32) * 4).astype(f16)
    q8, sq, cuq = O.quant_per_block_int8(q, cu_q, 128)
    k8, sk, cuk = O.quant_per_block_int8(k, cu_k, blkk)
    v8, sv, cuv = O.quant_per_block_int8(v, cu_k, blkk)
    return q, k, v, cu_q, cu_k, q8, sq.astype(f16), cuq, k8, sk.astype(f16), cuk, v8, sv.astype(f16), cuv


def check_int8_v_attention(Om):
    """INT8 route on int8 V codes (reference :449-497, INT8_USE_FP16_V = 0):
    fp64 attention over the dequantised scores and the dequantised V
    (v8 * sv of the key's BLKK block), with BLKK 64 (one V scale per tile,
    :472-481) and 16 (per-key V scales, :483-495).  Using the fp16 V in place of
    the codes moves the outputs by the V quantisation error (~0.05)."""
    for blkk in (64, 16):
        q, k, v, cu_q, cu_k, q8, sq16, cuq, k8, sk16, cuk, v8, sv16, cuv = _int8_v_setup(19, blkk)
        out = Om.attn_fwd(q, k, v, cu_q, cu_k, _all_bits(2, 3, ~np.uint64(0)), block_m=64, block_n_mask=64,
                          causal=True, routing_mode=O.ROUTING_INT8, q8=q8, k8=k8, sq16=sq16, sk16=sk16,
                          cu_q_scale=cuq, cu_k_scale=cuk, blkk=blkk, int8_use_fp16_v=False,
                          v8=v8, sv16=sv16, cu_v_scale=cuv)

        def scores(z, h):
            qa = q8[cu_q[z]:cu_q[z + 1], h].astype(np.float64)
            ka = k8[cu_k[z]:cu_k[z + 1], h // 2].astype(np.float64)
            lq, lk = qa.shape[0], ka.shape[0]
            rq = sq16[cuq[z] + np.arange(lq) // 128, h].astype(np.float64)
            rk = sk16[cuk[z] + np.arange(lk) // blkk, h // 2].astype(np.float64)
            return (qa @ ka.T) * rq[:, None] * rk[None, :] * 64 ** -0.5

        vdq = np.zeros(v.shape, np.float64)
        for z in range(2):
            for hk in range(2):
                keys = np.arange(cu_k[z + 1] - cu_k[z])
                s = sv16[cuv[z] + keys // blkk, hk].astype(np.float64)
                vdq[cu_k[z]:cu_k[z + 1], hk] = v8[cu_k[z]:cu_k[z + 1], hk].astype(np.float64) * s[:, None]
        ref = _fp64_attention(q, k, vdq, cu_q, cu_k, True, scores=scores)
        err = np.abs(out.astype(np.float64) - ref)
        # The bars of check_int8_attention scaled by the V magnitude (x4).
        assert err.max() < 1.6e-2 and err.mean() < 1.6e-3, (blkk, err.max(), err.mean())


def check_int8_v_known_answer(Om):
    """One row, two keys with given scores 0 and -s on the INT8 route with int8 V
    codes 0 and 100 (column 0) and V scale sv: m = 0, p0 = 1, p1 = fp16(2^-s),
    l = 1 + p1 (the row sum takes p, not p * sv), and PV takes p scaled in fp16
    (:472-481): out = fp16(fp16(p1 sv) 100 / (1 + p1)).  (s, sv) is the first
    pair of a fixed list for which leaving p sv unrounded gives another output."""
    L, d = 2, 16
    zeros8 = np.zeros((L, 1, d), np.int8)
    z16 = np.zeros((L, 1, d), f16)
    v8 = np.zeros((L, 1, d), np.int8)
    v8[1, 0, 0] = 100
    one = np.ones((1, 1), f16)
    cu = np.array([0, L])
    choice = None
    for s in (0.5, 0.75, 1.25, 1.5, 2.5):
        p1 = f32(f16(np.exp2(f32(-s))))
        for sv in (0.3, 0.37, 0.41, 0.53, 0.61, 0.77, 0.9):
            sv16 = f32(f16(sv))
            den = f32(f32(1) + p1)
            rounded = f16(f32(f32(f16(p1 * sv16)) * f32(100)) / den)
            unrounded = f16(f32(f32(p1 * sv16) * f32(100)) / den)
            if rounded != unrounded:
                choice = (s, sv, rounded)
                break
        if choice:
            break
    assert choice is not None
    s, sv, want = choice
    sc = np.array([[0.0, -s], [0.0, -s]], f16)
    out = Om.attn_fwd(z16, z16, z16, cu, cu, _all_bits(1, 1, 1), block_m=64, block_n_mask=64, causal=False,
                      routing_mode=O.ROUTING_INT8, q8=zeros8, k8=zeros8, sq16=one, sk16=one,
                      cu_q_scale=np.array([0, 1]), cu_k_scale=np.array([0, 1]), int8_use_fp16_v=False,
                      v8=v8, sv16=np.array([[sv]], f16), cu_v_scale=np.array([0, 1]),
                      qk16_override=lambda z, h: sc)
    assert out[0, 0, 0] == want and out[1, 0, 0] == want, (out[:, 0, 0], want, s, sv)


def check_bias_known_answer(Om):
    """One row, two keys with given fp16 scores 14.4375 and 0, bias 0 and 10,
    V = [0, 1] (column 0).  Reference :264-272: qk += fp16(b * LOG2E), where the
    fp16 bias times the Python constant computes in fp16, i.e. with LOG2E
    rounded to fp16 (1.4423828125): key 1's score is fp16(10 * 1.4423828125) =
    14.421875 (an fp32 LOG2E would give 14.4296875).  m = 14.4375, p0 = 1,
    p1 = fp16(2^(14.421875 - 14.4375)), out = fp16(p1 / (1 + p1))."""
    L, d = 2, 16
    z16 = np.zeros((L, 1, d), f16)
    v = np.zeros((L, 1, d), f16)
    v[1, 0, 0] = 1
    cu = np.array([0, L])
    sc = np.array([[14.4375, 0.0], [14.4375, 0.0]], f16)
    bias = np.zeros((1, 1, L, L), f16)
    bias[0, 0, :, 1] = 10
    assert f16(10 * f16(O.LOG2E)) == f16(14.421875) and f16(10 * O.LOG2E) == f16(14.4296875)
    p1 = f16(np.exp2(f32(f32(14.421875) - f32(14.4375))))
    want = f16(f32(p1) / f32(f32(1) + f32(p1)))
    out = Om.attn_fwd(z16, z16, v, cu, cu, _all_bits(1, 1, 0), block_m=64, block_n_mask=64, causal=False,
                      qk16_override=lambda z, h: sc, bias=bias)
    assert out[0, 0, 0] == want and out[1, 0, 0] == want, (out[:, 0, 0], want)


def check_bias_attention(Om):
    """Random bias on a causal GQA launch at both routes: fp64 softmax(q k^T sm +
    bias) v (a bias b in natural-log units is b * LOG2E in the kernel's base-2
    scores), within fp16 rounding of the bias term and the scores."""
    q, k, v, cu_q, cu_k = _inputs([96], 4, 2, 64, seed=23)
    rng = np.random.default_rng(29)
    bias = (rng.standard_normal((1, 4, 96, 96)) * 2).astype(f16)
    bias[0, :, 5, :] = 0
    q8, sq, cuq = O.quant_per_block_int8(q, cu_q, 128)
    k8, sk, cuk = O.quant_per_block_int8(k, cu_k, 64)
    sq16, sk16 = sq.astype(f16), sk.astype(f16)
    for mode in (O.ROUTING_FP16, O.ROUTING_INT8):
        out = Om.attn_fwd(q, k, v, cu_q, cu_k, _all_bits(2, 2, 0), block_m=64, block_n_mask=64, causal=True,
                          routing_mode=mode, q8=q8, k8=k8, sq16=sq16, sk16=sk16, cu_q_scale=cuq,
                          cu_k_scale=cuk, bias=bias)

        def scores(z, h):
            if mode == O.ROUTING_FP16:
                s = q[:, h].astype(np.float64) @ k[:, h // 2].astype(np.float64).T * 64 ** -0.5
            else:
                s = (q8[:, h].astype(np.float64) @ k8[:, h // 2].astype(np.float64).T
                     * sq16[0, h].astype(np.float64) * sk16[np.arange(96) // 64, h // 2].astype(np.float64)[None, :]
                     * 64 ** -0.5)
            return s + bias[0, h].astype(np.float64)

        ref = _fp64_attention(q, k, v, cu_q, cu_k, True, scores=scores)
        err = np.abs(out.astype(np.float64) - ref)
        assert err.max() < 1e-2 and err.mean() < 1e-3, (mode, err.max(), err.mean())


def check_bias_batch0(Om):
    """The reference reads the bias without a batch offset (:264-272: the
    pointer takes head, row and key strides, never stride_bz): every sequence of
    a packed launch adds bias[0].  Two sequences of 40 and 56 tokens: the second
    sequence's rows equal a launch of that sequence alone with bias[0], and
    differ from one with bias[1]."""
    q, k, v, cu_q, cu_k = _inputs([40, 56], 2, 1, 32, seed=31)
    rng = np.random.default_rng(37)
    bias = (rng.standard_normal((2, 2, 56, 56)) * 3).astype(f16)
    out = Om.attn_fwd(q, k, v, cu_q, cu_k, _all_bits(1, 1, 0), block_m=64, block_n_mask=64, causal=True,
                      bias=bias)
    cu1 = np.array([0, 56])
    sl = slice(40, 96)
    alone0 = Om.attn_fwd(q[sl], k[sl], v[sl], cu1, cu1, _all_bits(1, 1, 0), block_m=64, block_n_mask=64,
                         causal=True, bias=bias[:1])
    alone1 = Om.attn_fwd(q[sl], k[sl], v[sl], cu1, cu1, _all_bits(1, 1, 0), block_m=64, block_n_mask=64,
                         causal=True, bias=bias[1:])
    assert np.array_equal(out[sl], alone0)
    assert not np.array_equal(out[sl], alone1)


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
          check_int8_vector_scales, check_int8_v_attention, check_int8_v_known_answer, check_bias_known_answer,
          check_bias_attention, check_bias_batch0, check_route_table]


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
    # int8 V codes: the V scale dropped, fp16 V used on INT8 tiles, p * sv left unrounded
    "int8v_no_sv": ("p_sc = (p16.astype(f32) * sv[None, k0:k1].astype(f32)).astype(f16)", "p_sc = p16"),
    "int8v_fp16_v": ("pv8 = (p_sc.astype(f32) @ v8h[k0:k1])", "pv8 = (p_sc.astype(f32) @ vh[k0:k1])"),
    "int8v_unrounded_p_sv": ("p_sc = (p16.astype(f32) * sv[None, k0:k1].astype(f32)).astype(f16)",
                             "p_sc = (p16.astype(f32) * sv[None, k0:k1].astype(f32))"),
    # bias: LOG2E factor dropped, LOG2E taken in fp32, per-sequence bias, transposed bias
    "bias_no_log2e": ("bl = (b.astype(f32) * f32(f16(LOG2E))).astype(f16)", "bl = b"),
    "bias_fp32_log2e": ("bl = (b.astype(f32) * f32(f16(LOG2E))).astype(f16)",
                        "bl = (b.astype(f32) * f32(LOG2E)).astype(f16)"),
    "bias_batch_offset": ("np.asarray(bias)[0, h, :Lq, :Lk]", "np.asarray(bias)[min(z, len(bias) - 1), h, :Lq, :Lk]"),
    "bias_transposed": ("np.asarray(bias)[0, h, :Lq, :Lk]", "np.asarray(bias)[0, h, :Lk, :Lq].T"),
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
