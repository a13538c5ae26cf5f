"""CPU restatement of the TileMix prefill hot path -- TEST INFRASTRUCTURE ONLY.

This module is the checker, never the product: only tests/, the
``__graft_entry__.smoke()`` check and ``bench.py``'s ``cpu_baseline`` leg may
import it.  The product path (``tilemix_amd``) never imports it and fails
loudly when its HIP library is missing.

It is a numpy restatement (fp32 emulation with the reference's fp16 rounding
points) of:

* ``quant_per_block_int8``  <- attention/triton/quant_per_block_varlen.py:6-45
  (kernel) and :48-75 (scale bookkeeping of per_block_int8_single).
* ``attn_fwd``              <- attention/triton/tilemix.py:503-951 (kernel),
  :179-207 (online softmax), :210-300 (FP16 tile), :303-500 (INT8 tile),
  :1132-1337 (launch parameters: sm_scale default, scale layout).

Numerics contract (what the HIP kernel must reproduce):

1. qk_scale = fp32(sm_scale) * fp32(log2 e)                      (tilemix.py:641)
2. q16      = fp16(fp32(q) * qk_scale)                          (:643-649)
3. FP16 tile: qk = fp16(sum_d q16 k) -- the dot product accumulated wide and
   rounded once to fp16.  The reference accumulates this product in fp16
   (``out_dtype=tl.float16``, :254); no MI355X matrix instruction accumulates
   in fp16 (documented deviation).  The oracle accumulates in fp64 (exact for
   these operands up to 2^-53 relative) and rounds once; the kernel's fp32 MFMA
   accumulation may land one fp16 ulp away when the exact sum lies within a
   few fp32 ulps of an fp16 rounding midpoint.
4. INT8 tile: acc = sum_d q8 k8 (exact int32);  ss = fp16(fp32(fp16(sq sk)) qk_scale);
   qk = fp16(fp32(acc) fp32(ss))                                 (:380-404)
5. invalid (key >= Lk, or causal key > row + Lk - Lq) -> -inf     (:256-262)
6. online softmax per block_n-key tile (64, 128 or 256) in ascending key order:
   m' = max(m, max qk over the tile), p = fp16(exp2(qk - m')), l = l alpha +
   sum fp32(p), acc = acc alpha + p.V (fp32), alpha = exp2(m - m'); l starts at
   1.0                                                       (:179-207,727-729)
7. out = fp16(acc / l)                                           (:935-951)

Tiles beyond a query block's causal tile count are fully masked for every row
of that block, so processing them is an exact no-op: the oracle therefore runs
every row over every key tile with masking, which is the same arithmetic.

Parity pinning of each function (see tests/test_oracle.py):
* quant_per_block_int8: closed-form invariants (|code|<=127, argmax maps to
  +-127, round-half-away reconstruction bound), a brute-force scalar Python
  restatement on small blocks, tail / all-zero blocks.
* int32 accumulators: textbook integer GEMM (numpy int64).
* attention: at p=0 (all FP16) it reduces to causal softmax attention checked
  against an fp64 softmax(QK^T)V within fp16 rounding; a planted-mistake set
  (dropped 1/l, wrong causal offset, wrong GQA mapping, wrong route bit) must
  fail; INT8 route checked against the dequantised fp64 computation.
* int8 V codes (int8_use_fp16_v=False): fp64 attention over dequantised
  scores and dequantised V (BLKK 64 and 16) and a known answer in which the
  fp16 rounding of p * sv decides the output.
* bias: a known answer in which LOG2E taken at fp16 decides a score, fp64
  attention over scores + bias, and the batch-0 bias read in a two-sequence
  launch.
"""
from __future__ import annotations

import numpy as np

LOG2E = 1.4426950408889634
ROUTING_MIXED, ROUTING_FP16, ROUTING_INT8 = 0, 1, 2
BN = 64  # compute tile width in keys (block_n of the hot path)

f16 = np.float16
f32 = np.float32


def _ceil_div(a: int, b: int) -> int:
    return (a + b - 1) // b


# --------------------------------------------------------------------------
# quantisation
# --------------------------------------------------------------------------
def quant_per_block_int8(x: np.ndarray, cu_seqlens, blk: int, sm_scale: float = 1.0):
    """Per-(sequence, block of ``blk`` tokens, head) symmetric int8 quantisation.

    Follows attention/triton/quant_per_block_varlen.py:29-45 (kernel) and
    :52-63 (scale rows = exclusive cumsum of ceil(L_b / blk)).

    x: float16 [tokens, heads, dim].  Returns (codes int8 [tokens, heads, dim],
    scale float32 [rows, heads], cu_scale int64 [batch + 1]).  Tokens outside
    every sequence keep code 0.  An all-zero block (0/0 in the reference, whose
    result is undefined there) gets scale 0 and codes 0.
    """
    x = np.asarray(x)
    assert x.dtype == f16 and x.ndim == 3
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    lens = cu[1:] - cu[:-1]
    nblk = (lens + blk - 1) // blk
    cu_scale = np.concatenate([[0], np.cumsum(nblk)]).astype(np.int64)
    n_tok, heads, dim = x.shape
    codes = np.zeros((n_tok, heads, dim), dtype=np.int8)
    scale = np.zeros((int(cu_scale[-1]), heads), dtype=f32)
    s32 = f32(sm_scale)
    for b in range(len(lens)):
        L = int(lens[b])
        if L == 0:
            continue
        nb = int(nblk[b])
        xs = np.zeros((nb * blk, heads, dim), dtype=f32)
        xs[:L] = x[cu[b]:cu[b] + L].astype(f32) * s32             # :38-39
        blocks = xs.reshape(nb, blk, heads, dim)
        amax = np.abs(blocks).max(axis=(1, 3))                    # [nb, heads]
        s = (amax / f32(127.0)).astype(f32)                       # :40
        with np.errstate(divide="ignore", invalid="ignore"):
            t = (blocks / s[:, None, :, None]).astype(f32)        # :41
        t = (t + np.where(t >= 0, f32(0.5), f32(-0.5))).astype(f32)  # :42
        t = np.where(s[:, None, :, None] == 0, f32(0), t)
        c = np.trunc(t).astype(np.int64).astype(np.int8)          # :43
        codes[cu[b]:cu[b] + L] = c.reshape(nb * blk, heads, dim)[:L]
        scale[cu_scale[b]:cu_scale[b] + nb] = s
    return codes, scale, cu_scale


def quant_block_scalar(values, sm_scale: float = 1.0):
    """Element-by-element restatement of one block (brute force for tests)."""
    vals = [f32(f32(v) * f32(sm_scale)) for v in np.asarray(values, dtype=f16).reshape(-1)]
    amax = f32(0.0)
    for v in vals:
        if abs(v) > amax:
            amax = f32(abs(v))
    s = f32(amax / f32(127.0))
    out = []
    for v in vals:
        if s == 0:
            out.append(0)
            continue
        t = f32(v / s)
        t = f32(t + (f32(0.5) if t >= 0 else f32(-0.5)))
        out.append(int(t))  # int() truncates toward zero
    return np.array(out, dtype=np.int64), s


# --------------------------------------------------------------------------
# routing
# --------------------------------------------------------------------------
def route_table(bitmask, *, hk: int, Lq: int, Lk: int, block_m: int, block_n_mask: int,
                routing_mode: int) -> np.ndarray:
    """Route (True = INT8) of every (query block, 64-key tile) of one KV head.

    Row index hk * ceil(Lq / block_m) + m uses the per-sequence block count
    (attention/triton/tilemix.py:819-820); tile n reads bit n // (block_n_mask / 64)
    (:824-832).
    """
    mbz = _ceil_div(Lq, block_m)
    nt = _ceil_div(Lk, BN)
    if routing_mode == ROUTING_FP16:
        return np.zeros((mbz, nt), dtype=bool)
    if routing_mode == ROUTING_INT8:
        return np.ones((mbz, nt), dtype=bool)
    group = block_n_mask // BN
    bm = np.asarray(bitmask).astype(np.uint64)
    rows = bm[hk * mbz: hk * mbz + mbz]
    shifts = (np.arange(nt) // group).astype(np.uint64)
    return ((rows[:, None] >> shifts[None, :]) & np.uint64(1)).astype(bool)


# --------------------------------------------------------------------------
# attention
# --------------------------------------------------------------------------
def _scale_rows(scale16: np.ndarray, base: int, end: int, idx: np.ndarray, head: int) -> np.ndarray:
    """Clamped scale lookup (attention/triton/tilemix.py:380-387,671-698)."""
    if end <= base:
        return np.ones(idx.shape, dtype=f16)
    j = np.minimum(base + idx, end - 1)
    return scale16[j, head].astype(f16)


def fp16_tile_scores(q16: np.ndarray, k16: np.ndarray, accum: str = "exact") -> np.ndarray:
    """FP16 route scores fp16(dot(q16, k)) of attention/triton/tilemix.py:254, [Lq, Lk].

    The reference asks Triton for ``out_dtype=float16``; how its dot accumulates
    is the compiler's and the GPU's (unpinned: no reference output pins it).
    Three models of the sum over head_dim before the final fp16 rounding:

    * ``"exact"``: the exact sum, rounded once (the oracle's definition);
    * ``"fp32_k16"``: an fp32 accumulator updated once per 16-wide slice of
      head_dim in ascending order, each update the exact slice sum added with
      one fp32 rounding (the k-step order of the 32x32x16 f16 MFMA; the
      MFMA's internal summation of a k-step rounds differently, its fp32
      accumulators differ from this model by a few ulps on most entries, so
      this is a model of fp32 accumulation, not of the instruction's bits);
    * ``"fp16_k16"``: the same with an fp16 accumulator (a model of an
      fp16-accumulating matrix instruction per 16-wide slice).

    Products of two fp16 values are exact in fp64 and a 16-term slice sum is
    exact in fp64 unless its terms span more than ~27 binary orders of
    magnitude, which these inputs never reach.
    """
    if accum == "exact":
        return (q16.astype(np.float64) @ k16.astype(np.float64).T).astype(f16)
    if accum not in ("fp32_k16", "fp16_k16"):
        raise ValueError(f"unknown accumulation model {accum!r}")
    return k16_accumulate(q16, k16, f32 if accum == "fp32_k16" else f16).astype(f16)


def k16_accumulate(q16: np.ndarray, k16: np.ndarray, acc_dtype=f32) -> np.ndarray:
    """The accumulator of dot(q16, k16^T) updated once per 16-wide slice of
    head_dim (ascending), each update = exact slice sum added with one rounding
    to ``acc_dtype``; returned unrounded to fp16 ([Lq, Lk] of acc_dtype)."""
    qd = q16.astype(np.float64)
    kd = k16.astype(np.float64)
    acc = np.zeros((q16.shape[0], k16.shape[0]), dtype=acc_dtype)
    for d0 in range(0, q16.shape[1], 16):
        part = qd[:, d0:d0 + 16] @ kd[:, d0:d0 + 16].T
        acc = (acc.astype(np.float64) + part).astype(acc_dtype)
    return acc


def attn_fwd(q, k, v, cu_q, cu_k, bitmask, *, block_m: int, block_n_mask: int, causal: bool,
             sm_scale: float | None = None, routing_mode: int = ROUTING_MIXED,
             q8=None, k8=None, sq16=None, sk16=None, cu_q_scale=None, cu_k_scale=None,
             blkq: int = 128, blkk: int = 64, int8_use_fp16_v: bool = True,
             v8=None, sv16=None, cu_v_scale=None, bias=None, want_scores: bool = False,
             qk16_override=None, fp16_accum: str = "exact", block_n: int = 64):
    """fp32 emulation of attn_fwd over packed varlen [tokens, heads, dim] fp16 input.

    Returns out (float16, shape of q); with want_scores also a dict mapping
    (z, h) -> (qk_i32 [Lq, Lk] int64 (exact), qk16 [Lq, Lk] float16 pre-mask
    scores, route [Lq, Lk] bool).  ``qk16_override`` (callable (z, h) -> fp16
    [Lq, Lk] or None) replaces the score stage, so the softmax/PV stage can be
    checked on given scores.  ``fp16_accum`` is the accumulation of the FP16
    route's dot(q16, k) before its fp16 rounding (see ``fp16_tile_scores``).
    ``block_n`` is the key width of one online-softmax step (the reference's
    BLOCK_N, :603-615); route bits and K/V scales are per key, so it changes
    only where the running maximum is updated (block_n_mask % block_n == 0,
    :578-583).
    """
    if block_n % BN or block_n_mask % block_n:
        raise ValueError(f"block_n ({block_n}) must be a multiple of 64 dividing block_n_mask ({block_n_mask})")
    q = np.asarray(q)
    k = np.asarray(k)
    v = np.asarray(v)
    n_q, hq, dim = q.shape
    hkv = k.shape[1]
    group = hq // hkv
    if sm_scale is None:
        sm_scale = dim ** -0.5
    qk_scale = f32(f32(sm_scale) * f32(LOG2E))                       # :641
    cu_q = np.asarray(cu_q, dtype=np.int64)
    cu_k = np.asarray(cu_k, dtype=np.int64)
    out = np.zeros((n_q, hq, dim), dtype=f16)
    scores = {}
    need_int8 = routing_mode != ROUTING_FP16
    for z in range(len(cu_q) - 1):
        qs, Lq = int(cu_q[z]), int(cu_q[z + 1] - cu_q[z])
        ks, Lk = int(cu_k[z]), int(cu_k[z + 1] - cu_k[z])
        if Lq == 0:
            continue
        nt = _ceil_div(Lk, block_n)
        rows = np.arange(Lq)
        keys = np.arange(Lk)
        valid = np.broadcast_to(keys[None, :] < Lk, (Lq, Lk)).copy()
        if causal:
            valid &= keys[None, :] <= rows[:, None] + (Lk - Lq)            # :256-262
        for h in range(hq):
            hk = h // group
            route_mt = route_table(bitmask, hk=hk, Lq=Lq, Lk=Lk, block_m=block_m,
                                   block_n_mask=block_n_mask, routing_mode=routing_mode)
            route = np.repeat(np.repeat(route_mt, block_m, axis=0)[:Lq], BN, axis=1)[:, :Lk]
            qh = q[qs:qs + Lq, h].astype(f32)
            kh = k[ks:ks + Lk, hk].astype(f32)
            vh = v[ks:ks + Lk, hk].astype(f32)
            qk16 = np.zeros((Lq, Lk), dtype=f16)
            acc_i32 = None
            if not route.all():
                q16s = (qh * qk_scale).astype(f16)                           # :643-649
                s16 = fp16_tile_scores(q16s, kh.astype(f16), fp16_accum)      # :254
                qk16 = np.where(route, qk16, s16)
            if need_int8 and route.any():
                q8h = np.asarray(q8)[qs:qs + Lq, h].astype(np.float64)
                k8h = np.asarray(k8)[ks:ks + Lk, hk].astype(np.float64)
                acc_i32 = (q8h @ k8h.T).astype(np.int64)                     # :401 (exact)
                sq = _scale_rows(np.asarray(sq16), int(cu_q_scale[z]), int(cu_q_scale[z + 1]),
                                 rows // blkq, h)
                sk = _scale_rows(np.asarray(sk16), int(cu_k_scale[z]), int(cu_k_scale[z + 1]),
                                 keys // blkk, hk)
                sqk = (sq.astype(f32)[:, None] * sk.astype(f32)[None, :]).astype(f16)
                ss = (sqk.astype(f32) * qk_scale).astype(f16)                # :388/:398
                s8 = (acc_i32.astype(f32) * ss.astype(f32)).astype(f16)      # :402-404
                qk16 = np.where(route, s8, qk16)
            if qk16_override is not None:
                given = qk16_override(z, h)
                if given is not None:
                    qk16 = np.asarray(given, dtype=f16)
            s = np.where(valid, qk16.astype(f32), f32(-np.inf)).astype(f32)
            if bias is not None:
                b = np.asarray(bias)[0, h, :Lq, :Lk].astype(f16)            # no batch offset
                bl = (b.astype(f32) * f32(f16(LOG2E))).astype(f16)
                s = np.where(valid, (s.astype(f16).astype(f32) + bl.astype(f32)).astype(f16).astype(f32), s)
            if want_scores:
                scores[(z, h)] = (acc_i32, qk16, route)
            # ---- online softmax, one block_n-key tile at a time -------------
            m_i = np.full(Lq, -np.inf, dtype=f32)
            l_i = np.ones(Lq, dtype=f32)
            acc = np.zeros((Lq, dim), dtype=f32)
            if not int8_use_fp16_v and need_int8:
                v8h = np.asarray(v8)[ks:ks + Lk, hk].astype(f32)
                sv = _scale_rows(np.asarray(sv16), int(cu_v_scale[z]), int(cu_v_scale[z + 1]),
                                 keys // blkk, hk)
            for n in range(nt):
                k0, k1 = n * block_n, min((n + 1) * block_n, Lk)
                st = s[:, k0:k1]
                mx = st.max(axis=1)
                has = mx != -np.inf
                m_next = np.where(has, np.maximum(m_i, mx), m_i).astype(f32)
                with np.errstate(invalid="ignore"):
                    shifted = np.where(has[:, None], st - m_next[:, None], f32(-np.inf)).astype(f32)
                    alpha = np.where(has, np.exp2(m_i - m_next), f32(1.0)).astype(f32)
                p16 = np.exp2(shifted).astype(f32).astype(f16)
                l_tile = p16.astype(f32).sum(axis=1, dtype=f32)
                acc = (acc * alpha[:, None]).astype(f32)
                l_i = (l_i * alpha + l_tile).astype(f32)
                m_i = m_next
                if not int8_use_fp16_v and need_int8:
                    r8 = route[:, k0:k1]
                    p_sc = (p16.astype(f32) * sv[None, k0:k1].astype(f32)).astype(f16)
                    pv16 = (p16.astype(f32) @ vh[k0:k1]).astype(f32)
                    pv8 = (p_sc.astype(f32) @ v8h[k0:k1]).astype(f32)
                    # route is uniform over a tile row-block: pick per row
                    acc = acc + np.where(r8[:, :1], pv8, pv16)
                else:
                    acc = acc + (p16.astype(f32) @ vh[k0:k1]).astype(f32)
            out[qs:qs + Lq, h] = (acc / l_i[:, None]).astype(f16)
    if want_scores:
        return out, scores
    return out


def make_inputs_dense(B: int, Hq: int, Hk: int, L: int, D: int, seed: int = 0,
                      outlier_channels=(), outlier_scale: float = 8.0, head_scale=None):
    """Seeded fp16 q [B*L, Hq, D], k, v [B*L, Hk, D] ~ N(0,1) (numpy generator).

    ``outlier_channels`` are multiplied by ``outlier_scale`` in Q and K before
    the fp16 cast; ``head_scale`` (per KV... per head arrays) multiplies heads.
    """
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B * L, Hq, D), dtype=np.float32)
    k = rng.standard_normal((B * L, Hk, D), dtype=np.float32)
    v = rng.standard_normal((B * L, Hk, D), dtype=np.float32)
    for c in outlier_channels:
        q[:, :, c] *= outlier_scale
        k[:, :, c] *= outlier_scale
    if head_scale is not None:
        hs_q, hs_k = head_scale
        q *= np.asarray(hs_q, dtype=np.float32)[None, :, None]
        k *= np.asarray(hs_k, dtype=np.float32)[None, :, None]
        v *= np.asarray(hs_k, dtype=np.float32)[None, :, None]
    return q.astype(f16), k.astype(f16), v.astype(f16)
