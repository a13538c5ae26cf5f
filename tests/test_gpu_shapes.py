"""GPU parity of the launch shapes beyond block_n = 64 / BLKK = 64 / head_dim % 16 == 0.

* block_n 128 and 256 (reference configs (64, 128), (64, 256) and any
  block_m with the fallback config, attention/triton/tilemix.py:19-38,
  1049-1080): one online-softmax step per block_n keys, in every kernel kind
  (32-row, split 32-row, 16-row) and routing mode, fp16 and int8 V;
* K/V scale blocks BLKK of 16, 32 and 48 keys (the per-key lookup
  sk[key // BLKK], :390, :485), with the INT8 scores checked bit for bit
  through the score dump;
* head_dims that are not multiples of 16 (24, 40, 72, 100, 120, 127): the
  host layer zero-pads Q/K/V to the next multiple of 16, the reference masks
  the columns past head_dim (:252, :364, :639);
* block_m 256 and 512 (the reference's fallback sizes), bias on the GEN
  kernels, and Q/K/V views whose strides exceed the kernel's 2 GiB buffer
  span.

All against the CPU oracle at the full bar (max-abs 2e-3, mean-abs 2e-4).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import tilemix_oracle as O
from tests._helpers import assert_close_out, bitmask_tensor, packed_inputs, random_bitmask, to_dev
from tilemix_amd.attention.hip import tilemix as tmx

pytestmark = pytest.mark.gpu

MODES = {"mixed": 0, "fp16": 1, "int8": 2}


def _case(device, lengths, hq, hk, d, block_m, block_n, bnm, causal, mode, int8v, seed, blkk=64, blkq=128,
          outliers=(), bias=None):
    """Launch through tilemix_attention_with_quant and run the oracle on the same inputs."""
    q, k, v, cu = packed_inputs(lengths, hq, hk, d, seed=seed, outliers=outliers)
    max_len = max(lengths)
    bits = random_bitmask(hk, -(-max_len // block_m), seed)
    print(f"case lengths={lengths} hq={hq} hk={hk} d={d} block_m={block_m} block_n={block_n} bnm={bnm} "
          f"causal={causal} mode={mode} int8_use_fp16_v={int8v} BLKK={blkk} seed={seed} "
          f"bias={bias is not None}", flush=True)
    out, mode_ret = tmx.tilemix_attention_with_quant(
        to_dev(q, device), to_dev(k, device), to_dev(v, device), to_dev(cu, device), to_dev(cu, device),
        max_len, max_len, bitmask_tensor(bits, device), block_m=block_m, block_n=block_n, block_n_mask=bnm,
        BLKQ=blkq, BLKK=blkk, causal=causal, routing_mode=mode, scalar_scales=False, int8_use_fp16_v=int8v,
        bias=None if bias is None else to_dev(bias, device))
    torch.cuda.synchronize()
    assert mode_ret == mode
    q8, sq, cuq = O.quant_per_block_int8(q, cu, blkq)
    k8, sk, cuk = O.quant_per_block_int8(k, cu, blkk)
    extra = {}
    if not int8v:
        v8, sv, cuv = O.quant_per_block_int8(v, cu, blkk)
        extra = dict(v8=v8, sv16=sv.astype(np.float16), cu_v_scale=cuv)
    ref = O.attn_fwd(q, k, v, cu, cu, bits, block_m=block_m, block_n_mask=bnm, causal=causal,
                     routing_mode=MODES[mode], q8=q8, k8=k8, sq16=sq.astype(np.float16), sk16=sk.astype(np.float16),
                     cu_q_scale=cuq, cu_k_scale=cuk, blkq=blkq, blkk=blkk, int8_use_fp16_v=int8v,
                     block_n=block_n, bias=bias, **extra)
    return out.cpu().numpy(), ref


# name, lengths, hq, hk, d, block_m, block_n, block_n_mask, causal, mode, int8_use_fp16_v
BLOCK_N_CASES = [
    # the reference's (64, 128) / (64, 256) configs: split 32-row kernel (mixed,
    # fp16 V), 16-row kernel (mixed, int8 V), 32-row kernel (fp16 / int8 modes)
    ("bm64_bn128_mixed", [300, 129, 1], 4, 2, 128, 64, 128, 128, True, "mixed", True),
    ("bm64_bn256_mixed", [600, 70], 4, 2, 128, 64, 256, 256, True, "mixed", True),
    ("bm64_bn128_mixed_int8v", [300, 129], 4, 2, 128, 64, 128, 256, True, "mixed", False),
    ("bm64_bn256_mixed_int8v_d64", [520, 33], 4, 1, 64, 64, 256, 256, True, "mixed", False),
    ("bm64_bn128_fp16", [333, 64], 4, 2, 128, 64, 128, 128, True, "fp16", True),
    ("bm64_bn256_int8", [333, 64], 4, 2, 128, 64, 256, 256, True, "int8", True),
    ("bm64_bn128_int8_int8v", [250], 4, 2, 64, 64, 128, 128, True, "int8", False),
    # block_m 128 (reference fallback config), non-causal, mask groups of 2 tiles
    ("bm128_bn128_mixed", [700, 200], 6, 2, 128, 128, 128, 256, True, "mixed", True),
    ("bm128_bn256_mixed_int8v", [700], 4, 2, 128, 128, 256, 256, True, "mixed", False),
    ("bm128_bn128_noncausal_d64", [300, 100], 4, 2, 64, 128, 128, 128, False, "mixed", True),
    ("bm64_bn256_noncausal", [400, 77], 2, 1, 128, 64, 256, 512, False, "mixed", True),
]


@pytest.mark.parametrize("case", BLOCK_N_CASES, ids=[c[0] for c in BLOCK_N_CASES])
def test_block_n_matches_oracle(device, case):
    name, lengths, hq, hk, d, block_m, block_n, bnm, causal, mode, int8v = case
    got, ref = _case(device, lengths, hq, hk, d, block_m, block_n, bnm, causal, mode, int8v, seed=51)
    assert_close_out(got, ref)


def test_block_n_changes_the_result(device):
    """block_n is not a tiling detail: the same inputs at block_n 64 and 128
    give different outputs (the p values are rounded against different
    maxima), and each matches the oracle of its own block_n."""
    args = (device, [512], 4, 2, 128, 64)
    got64, ref64 = _case(*args, 64, 128, True, "fp16", True, seed=52)
    got128, ref128 = _case(*args, 128, 128, True, "fp16", True, seed=52)
    assert_close_out(got64, ref64)
    assert_close_out(got128, ref128)
    assert not np.array_equal(ref64, ref128)
    assert not np.array_equal(got64, got128)


# block_m 256 / 512 (the reference's fallback sizes, models/tilemix_llama.py:137-140,
# launched with the fallback config, attention/triton/tilemix.py:1074-1084): 128-row
# workgroups that read the routing row of the block holding them.
# name, lengths, hq, hk, d, block_m, block_n, block_n_mask, causal, mode, int8_use_fp16_v
BLOCK_M_LARGE_CASES = [
    ("bm256_mixed", [700, 129, 1], 4, 2, 128, 256, 64, 64, True, "mixed", True),
    ("bm512_mixed", [1200, 300], 4, 2, 128, 512, 64, 128, True, "mixed", True),
    ("bm256_mixed_int8v", [700, 200], 4, 2, 128, 256, 64, 64, True, "mixed", False),
    ("bm512_mixed_int8v_d64", [900], 4, 1, 64, 512, 64, 64, True, "mixed", False),
    ("bm256_bn128_mixed", [600, 77], 4, 2, 128, 256, 128, 256, True, "mixed", True),
    ("bm256_int8", [333], 4, 2, 128, 256, 64, 64, True, "int8", True),
    ("bm512_noncausal", [520, 40], 2, 1, 128, 512, 64, 64, False, "mixed", True),
]


@pytest.mark.parametrize("case", BLOCK_M_LARGE_CASES, ids=[c[0] for c in BLOCK_M_LARGE_CASES])
def test_block_m_256_512_matches_oracle(device, case):
    name, lengths, hq, hk, d, block_m, block_n, bnm, causal, mode, int8v = case
    got, ref = _case(device, lengths, hq, hk, d, block_m, block_n, bnm, causal, mode, int8v, seed=57)
    assert_close_out(got, ref)


def test_block_m_256_reads_its_blocks_routing_row(device):
    """block_m 256 and 128 on the same inputs and one routing pattern per
    256 rows: the block_m 256 launch with map row j equals the block_m 128
    launch whose rows 2j and 2j + 1 both hold row j (bit for bit), and differs
    from one that takes the rows unexpanded."""
    lengths, hq, hk, d = [700], 4, 2, 128
    q, k, v, cu = packed_inputs(lengths, hq, hk, d, seed=58)
    bits256 = random_bitmask(hk, 3, 58)
    bits128 = np.repeat(bits256.reshape(hk, 3), 2, axis=1)[:, :6].reshape(-1)
    dev = lambda a: to_dev(a, device)  # noqa: E731
    outs = {}
    for name, bm, bits in (("256", 256, bits256), ("128", 128, bits128),
                           ("128_unexpanded", 128, np.resize(bits256, hk * 6))):
        outs[name], _ = tmx.tilemix_attention_with_quant(
            dev(q), dev(k), dev(v), dev(cu), dev(cu), 700, 700, bitmask_tensor(bits, device), block_m=bm,
            block_n=64, causal=True, routing_mode="mixed", scalar_scales=False, int8_use_fp16_v=True)
    torch.cuda.synchronize()
    assert torch.equal(outs["256"], outs["128"])
    assert not torch.equal(outs["256"], outs["128_unexpanded"])


# Bias on the GEN kernels (block_n 128 / 256, or BLKK not a multiple of 64):
# the masked max pass and the update pass both add it.
# name, lengths, hq, hk, d, block_m, block_n, block_n_mask, mode, int8_use_fp16_v, BLKK
GEN_BIAS_CASES = [
    ("bn128_mixed_bm128", [300, 129], 4, 2, 128, 128, 128, 128, "mixed", True, 64),
    ("bn256_mixed_bm64_int8v", [400, 100], 4, 2, 128, 64, 256, 256, "mixed", False, 64),
    ("bn128_mixed_bm64_split", [333, 64], 4, 2, 128, 64, 128, 128, "mixed", True, 64),
    ("blkk32_int8_bm128_int8v", [300], 4, 2, 128, 128, 64, 128, "int8", False, 32),
    ("blkk32_bn128_mixed_bm64_int8v", [333, 64], 4, 2, 128, 64, 128, 128, "mixed", False, 32),
    ("bn256_fp16_bm128_d64", [520], 2, 1, 64, 128, 256, 256, "fp16", True, 64),
]


@pytest.mark.parametrize("case", GEN_BIAS_CASES, ids=[c[0] for c in GEN_BIAS_CASES])
def test_gen_bias_matches_oracle(device, case):
    """Additive fp16 bias (reference :264-272, batch-0 bias for every sequence)
    through the GEN kernels, fp16 and int8 V, against the oracle."""
    name, lengths, hq, hk, d, block_m, block_n, bnm, mode, int8v, blkk = case
    rng = np.random.default_rng(59)
    bias = (rng.standard_normal((len(lengths), hq, max(lengths), max(lengths))) * 2).astype(np.float16)
    got, ref = _case(device, lengths, hq, hk, d, block_m, block_n, bnm, True, mode, int8v, seed=59, blkk=blkk,
                     bias=bias)
    assert_close_out(got, ref)


def test_kv_span_beyond_2gib(device):
    """Q, K and V as views into one buffer with a 16 MiB token stride: (max_seqlen_k
    + 64) K/V token strides and 128 Q token strides exceed the kernel's 2 GiB
    buffer span, so the host passes head-major copies (token stride head_dim).
    The output equals the launch on dense copies bit for bit and matches the
    oracle (the reference addresses any strides with 64-bit pointers,
    attention/triton/tilemix.py:1259-1275)."""
    lengths, hq, hk, d = [300, 129], 4, 2, 128
    q, k, v, cu = packed_inputs(lengths, hq, hk, d, seed=60)
    n = sum(lengths)
    stride = 8 << 20  # elements per token: 16 MiB
    buf = torch.empty((n, stride), dtype=torch.float16, device=device)
    cols = [(0, hq), (hq, hk), (hq + hk, hk)]
    views = [buf.as_strided((n, h, d), (stride, d, 1), c0 * d) for c0, h in cols]
    for view, a in zip(views, (q, k, v)):
        view.copy_(to_dev(a, device))
    qv, kv, vv = views
    assert not tmx._span_fits(kv, 300 + 64) and not tmx._span_fits(qv, 128)
    max_len = max(lengths)
    bits = random_bitmask(hk, -(-max_len // 128), 60)
    print(f"span case lengths={lengths} token stride={stride * 2} bytes", flush=True)
    kw = dict(block_m=128, block_n=64, causal=True, routing_mode="mixed", scalar_scales=True,
              int8_use_fp16_v=True)
    cud, bmd = to_dev(cu, device), bitmask_tensor(bits, device)
    out_view, _ = tmx.tilemix_attention_with_quant(qv, kv, vv, cud, cud, max_len, max_len, bmd, **kw)
    out_dense, _ = tmx.tilemix_attention_with_quant(qv.contiguous(), kv.contiguous(), vv.contiguous(), cud, cud,
                                                    max_len, max_len, bmd, **kw)
    torch.cuda.synchronize()
    del buf, views, qv, kv, vv
    assert torch.equal(out_view, out_dense)
    q8, sq, cuq = O.quant_per_block_int8(q, cu, 128)
    k8, sk, cuk = O.quant_per_block_int8(k, cu, 64)
    ref = O.attn_fwd(q, k, v, cu, cu, bits, block_m=128, block_n_mask=64, causal=True, q8=q8, k8=k8,
                     sq16=sq.astype(np.float16), sk16=sk.astype(np.float16), cu_q_scale=cuq, cu_k_scale=cuk)
    assert_close_out(out_view.cpu().numpy(), ref)


# name, lengths, hq, hk, d, block_m, block_n, mode, int8_use_fp16_v, BLKK
BLKK_CASES = [
    ("blkk16_int8_bm128", [300, 129], 4, 2, 128, 128, 64, "int8", True, 16),
    ("blkk32_mixed_bm128_int8v", [300], 4, 2, 128, 128, 64, "mixed", False, 32),
    ("blkk16_mixed_bm64_split", [333, 64], 4, 2, 128, 64, 64, "mixed", True, 16),
    ("blkk32_mixed_bm64_int8v", [333, 64], 4, 2, 128, 64, 64, "mixed", False, 32),
    ("blkk48_int8_bm64_int8v_d64", [250, 97], 4, 1, 64, 64, 64, "int8", False, 48),
    ("blkk32_bn128_mixed_bm64", [400], 4, 2, 128, 64, 128, "mixed", True, 32),
    ("blkk128_bn256_int8", [600], 4, 2, 128, 128, 256, "int8", False, 128),
]


@pytest.mark.parametrize("case", BLKK_CASES, ids=[c[0] for c in BLKK_CASES])
def test_blkk_matches_oracle(device, case):
    name, lengths, hq, hk, d, block_m, block_n, mode, int8v, blkk = case
    got, ref = _case(device, lengths, hq, hk, d, block_m, block_n, max(block_n, 128), True, mode, int8v,
                     seed=53, blkk=blkk)
    assert_close_out(got, ref)


@pytest.mark.parametrize("block_m,block_n,blkk", [(64, 64, 16), (128, 64, 32), (64, 128, 48), (128, 256, 16)])
def test_gen_scores_bitexact(device, block_m, block_n, blkk):
    """Score dump of the GEN kernels: INT8-routed int32 accumulators and fp16
    scores bit for bit against the oracle (per-key K scales, both passes of a
    block_n tile write the same scores); softmax + PV checked on the kernel's
    own scores."""
    lengths, hq, hk, d = [300, 129], 4, 2, 128
    q, k, v, cu = packed_inputs(lengths, hq, hk, d, seed=54, outliers=(1, 9))
    max_len = max(lengths)
    bnm = max(block_n, 128)
    bits = random_bitmask(hk, -(-max_len // block_m), 54)
    q8, sq, cuq = O.quant_per_block_int8(q, cu, 128)
    k8, sk, cuk = O.quant_per_block_int8(k, cu, blkk)
    print(f"dump block_m={block_m} block_n={block_n} BLKK={blkk}", flush=True)
    out, qk_i32, qk16 = tmx.debug_launch(
        to_dev(q, device), to_dev(k, device), to_dev(v, device), to_dev(cu, device), to_dev(cu, device),
        max_len, max_len, bitmask_tensor(bits, device), q8=to_dev(q8, device), k8=to_dev(k8, device),
        sQ_blocks=to_dev(sq.astype(np.float16), device), sK_blocks=to_dev(sk.astype(np.float16), device),
        cu_q_scale=to_dev(cuq.astype(np.int32), device), cu_k_scale=to_dev(cuk.astype(np.int32), device),
        block_m=block_m, block_n=block_n, block_n_mask=bnm, BLKK=blkk, causal=True, routing_mode="mixed")
    torch.cuda.synchronize()
    kw = dict(block_m=block_m, block_n_mask=bnm, causal=True, routing_mode=0, q8=q8, k8=k8,
              sq16=sq.astype(np.float16), sk16=sk.astype(np.float16), cu_q_scale=cuq, cu_k_scale=cuk, blkk=blkk,
              block_n=block_n)
    _, scores = O.attn_fwd(q, k, v, cu, cu, bits, want_scores=True, **kw)
    gi, gf = qk_i32.cpu().numpy(), qk16.cpu().numpy()
    n_int8 = 0
    dumped = {}
    for (z, h), (acc, s16, route) in scores.items():
        qs, L = int(cu[z]), int(cu[z + 1] - cu[z])
        valid = np.arange(L)[None, :] <= np.arange(L)[:, None]
        sel = valid & route
        n_int8 += int(sel.sum())
        np.testing.assert_array_equal(gi[qs:qs + L, h, :L][sel], acc[sel].astype(np.int32))
        np.testing.assert_array_equal(gf[qs:qs + L, h, :L][sel].view(np.uint16), s16[sel].view(np.uint16))
        dumped[(z, h)] = gf[qs:qs + L, h, :L]
    assert n_int8 > 0
    ref_given = O.attn_fwd(q, k, v, cu, cu, bits, qk16_override=lambda z, h: dumped[(z, h)], **kw)
    assert_close_out(out.cpu().numpy(), ref_given)


# name, lengths, hq, hk, d, block_m, mode, int8_use_fp16_v
HEAD_DIM_CASES = [
    ("d72_mixed_bm128", [300, 129], 4, 2, 72, 128, "mixed", True),
    ("d100_int8_bm64", [250, 64], 4, 2, 100, 64, "int8", True),
    ("d24_fp16_bm64", [200], 4, 1, 24, 64, "fp16", True),
    ("d40_mixed_bm64_int8v", [333], 4, 2, 40, 64, "mixed", False),
    ("d120_mixed_bm64", [300, 1], 4, 2, 120, 64, "mixed", True),
    ("d127_int8_bm128_int8v", [257], 2, 1, 127, 128, "int8", False),
]


@pytest.mark.parametrize("case", HEAD_DIM_CASES, ids=[c[0] for c in HEAD_DIM_CASES])
def test_head_dim_padding_matches_oracle(device, case):
    """Any head_dim <= 128: the host zero-pads to a multiple of 16; the output
    keeps the caller's width and sm_scale defaults to the original head_dim."""
    name, lengths, hq, hk, d, block_m, mode, int8v = case
    got, ref = _case(device, lengths, hq, hk, d, block_m, 64, 64, True, mode, int8v, seed=55)
    assert got.shape[-1] == d
    assert_close_out(got, ref)


def test_head_dim_padding_prequantized(device):
    """launch_prequantized with codes of the caller's width (72): Q/K/V and
    q8/k8/v8 are padded together; the output buffer passed in is filled."""
    lengths, hq, hk, d = [200, 64], 4, 2, 72
    q, k, v, cu = packed_inputs(lengths, hq, hk, d, seed=56)
    q8, sq, cuq = O.quant_per_block_int8(q, cu, 128)
    k8, sk, cuk = O.quant_per_block_int8(k, cu, 64)
    v8, sv, cuv = O.quant_per_block_int8(v, cu, 64)
    bits = random_bitmask(hk, 4, 56)
    dev = lambda a: to_dev(a, device)  # noqa: E731
    o = torch.empty((sum(lengths), hq, d), dtype=torch.float16, device=device)
    out, mode = tmx.launch_prequantized(
        dev(q), dev(k), dev(v), dev(cu), dev(cu), 200, 200, bitmask_tensor(bits, device),
        q8=dev(q8), k8=dev(k8), v8=dev(v8), sQ_blocks=dev(sq.astype(np.float16)),
        sK_blocks=dev(sk.astype(np.float16)), sV_blocks=dev(sv.astype(np.float16)),
        cu_q_scale=dev(cuq.astype(np.int32)), cu_k_scale=dev(cuk.astype(np.int32)),
        cu_v_scale=dev(cuv.astype(np.int32)), block_m=64, block_n=64, block_n_mask=64, causal=True,
        routing_mode="mixed", scalar_scales=False, int8_use_fp16_v=False, o=o)
    torch.cuda.synchronize()
    assert out is o and mode == "mixed"
    ref = O.attn_fwd(q, k, v, cu, cu, bits, block_m=64, block_n_mask=64, causal=True, q8=q8, k8=k8,
                     sq16=sq.astype(np.float16), sk16=sk.astype(np.float16), cu_q_scale=cuq, cu_k_scale=cuk,
                     int8_use_fp16_v=False, v8=v8, sv16=sv.astype(np.float16), cu_v_scale=cuv)
    assert_close_out(o.cpu().numpy(), ref)


@pytest.mark.parametrize("seed", range(16))
def test_random_wide_configurations(device, seed):
    """Seeded random draws over the widened launch space: block_n 64/128/256,
    BLKK 16/32/64/128, head_dim 32..128 (any width), block_m 64/128, mask
    groups of 1-2 block_n tiles, causal or not, mixed/fp16/int8 routing, fp16
    or int8 V."""
    rng = np.random.default_rng(3000 + seed)
    n_seq = int(rng.integers(1, 4))
    lengths = [int(x) for x in rng.integers(1, 701, n_seq)]
    hq, hk = [(4, 1), (4, 2), (6, 2), (8, 8), (6, 3)][int(rng.integers(0, 5))]
    d = int(rng.integers(32, 129))
    block_m = [64, 128][int(rng.integers(0, 2))]
    block_n = [64, 128, 256][int(rng.integers(0, 3))]
    bnm = block_n * int(rng.integers(1, 3))
    if -(-max(lengths) // bnm) > 64:
        bnm = block_n * 2
    blkk = [16, 32, 64, 128][int(rng.integers(0, 4))]
    causal = bool(rng.integers(0, 4))
    mode = ["mixed", "mixed", "fp16", "int8"][int(rng.integers(0, 4))]
    int8v = True if mode == "fp16" else bool(rng.integers(0, 2))
    got, ref = _case(device, lengths, hq, hk, d, block_m, block_n, bnm, causal, mode, int8v, seed=4000 + seed,
                     blkk=blkk)
    assert_close_out(got, ref)
