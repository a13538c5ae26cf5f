"""The pipelined assembly tile loop (attn_pipe_asm.h) against the C++ tile body
of the same kernel, bit for bit, and against the oracle.

TILEMIX_HIP_PIPE=0 makes the launcher run the C++ tile body for every tile;
by default the head_dim > 64, 128-row-workgroup launches on fp16 V without
bias run their unmasked tiles through the assembly loop.  The cases cover the
loop's boundaries: sequences shorter than one tile (no pipelined tile), one
and two pipelined tiles (FILL then DRAIN at once), odd and even counts (both
unrolled parities end the loop), ragged and empty sequences in one launch,
the causal diagonal and a ragged end handed to the C++ body, Lq != Lk, mask
groups of two tiles, block_m 256 (routing rows shared by two workgroups),
block_m 64 with mixed routing (split workgroups: the two 64-row halves route
separately, and a tile past the low half's last key copies only the high
half's K format),
head_dim 80 and 96 (zero-padded columns), MHA and GQA 4, each routing mode,
and the INT8 scale bookkeeping at BLKK 128 / 256 (scale blocks spanning tiles).
"""
import os

import numpy as np
import pytest

from oracle import tilemix_oracle as O
from tests._helpers import assert_close_out, bitmask_tensor, packed_inputs, random_bitmask, to_dev
from tilemix_amd.attention import precision_maps as pm
from tilemix_amd.attention.hip import tilemix as tmx

pytestmark = pytest.mark.gpu

# name, q lengths, k lengths (None: same), hq, hk, d, block_m, block_n_mask, causal, mode, map, blkk
CASES = [
    ("short_and_ragged", [1, 50, 63, 64, 65, 127, 128, 129, 191, 257, 0, 300], None, 4, 2, 128, 128, 64, True,
     "mixed", "rand", 64),
    ("one_two_three_tiles_noncausal", [64, 128, 192, 256, 100], None, 2, 1, 128, 128, 64, False, "mixed", "rand",
     64),
    ("long_causal_mixed", [1024, 777], None, 6, 2, 128, 128, 64, True, "mixed", "rand", 64),
    ("long_causal_fp16", [1024, 777], None, 6, 2, 128, 128, 64, True, "fp16", "rand", 64),
    ("long_causal_int8", [1024, 777], None, 6, 2, 128, 128, 64, True, "int8", "rand", 64),
    ("sptrans", [2048], None, 3, 1, 128, 128, 64, True, "mixed", "sptrans", 64),
    ("lq_lt_lk", [100, 300, 64], [400, 1000, 64], 4, 2, 128, 128, 64, True, "mixed", "rand", 64),
    ("lq_gt_lk", [600, 300], [200, 299], 4, 2, 128, 128, 64, True, "mixed", "rand", 64),
    ("noncausal_ragged_lk", [300, 450], [333, 513], 2, 2, 128, 128, 64, False, "mixed", "rand", 64),
    ("mask_group2", [900], None, 4, 1, 128, 128, 128, True, "mixed", "rand", 64),
    ("block_m_256", [700, 300], None, 4, 2, 128, 256, 64, True, "mixed", "rand", 64),
    ("hd80_mha", [500], None, 3, 3, 80, 128, 64, True, "mixed", "rand", 64),
    ("hd96_gqa4", [640], None, 8, 2, 96, 128, 64, True, "mixed", "rand", 64),
    ("blkk128", [900, 130], None, 4, 2, 128, 128, 64, True, "mixed", "rand", 128),
    ("blkk256_int8", [1000], None, 2, 1, 128, 128, 64, True, "int8", "rand", 256),
    ("fp16_bm64", [333, 64], None, 4, 2, 128, 64, 64, True, "fp16", "rand", 64),
    # block_m 64 with mixed routing: split workgroups (per-half routes, both K formats per stage)
    ("split_sptrans", [2048], None, 3, 1, 128, 64, 64, True, "mixed", "sptrans", 64),
    ("split_short_and_ragged", [1, 63, 64, 65, 127, 129, 191, 257, 0, 700], None, 4, 2, 128, 64, 64, True,
     "mixed", "rand", 64),
    ("split_lq_lt_lk", [100, 300, 64], [400, 1000, 64], 4, 2, 128, 64, 64, True, "mixed", "rand", 64),
    ("split_lq_gt_lk", [600, 300], [200, 299], 4, 2, 128, 64, 64, True, "mixed", "rand", 64),
    ("split_noncausal", [300, 450], [333, 513], 2, 2, 128, 64, 64, False, "mixed", "rand", 64),
    ("split_group2_blkk128", [900, 130], None, 4, 2, 128, 64, 128, True, "mixed", "rand", 128),
    ("split_hd96_gqa3", [640], None, 6, 2, 96, 64, 64, True, "mixed", "rand", 64),
]


def _max_len(lq, lk):
    # the launch takes one max length for Q and K (packed routing)
    return max(max(lq), max(lk or lq))


def _bits(kind, lq, lk, hk, block_m, bnm, seed):
    m_blocks = -(-_max_len(lq, lk) // block_m)
    if kind == "rand":
        return random_bitmask(hk, m_blocks, seed)
    row = pm.make_precision_bitmask(_max_len(lq, lk), block_m, bnm, None, percentage=0.5, pattern_type="sptrans",
                                    pattern_params={"stride": 128, "c": 32}, COMPUTE_BLOCK_N=64)
    return np.array([int(x) for x in row.tolist()] * hk, dtype=np.uint64)


def _launch(device, inputs, case, pipe):
    name, lq, lk, hq, hk, d, block_m, bnm, causal, mode, kind, blkk = case
    q, k, v, cuq, cuk, bits = inputs
    old = os.environ.get("TILEMIX_HIP_PIPE")
    os.environ["TILEMIX_HIP_PIPE"] = "1" if pipe else "0"
    try:
        out, _ = tmx.tilemix_attention_with_quant(
            to_dev(q, device), to_dev(k, device), to_dev(v, device), to_dev(cuq, device), to_dev(cuk, device),
            _max_len(lq, lk), _max_len(lq, lk), bitmask_tensor(bits, device), block_m=block_m, block_n=64,
            block_n_mask=bnm, BLKQ=128, BLKK=blkk, causal=causal, routing_mode=mode,
            scalar_scales=(block_m == 128 and blkk == 64),
            int8_use_fp16_v=True)
        return out.cpu().numpy()
    finally:
        if old is None:
            del os.environ["TILEMIX_HIP_PIPE"]
        else:
            os.environ["TILEMIX_HIP_PIPE"] = old


def _inputs(case, seed, outliers=()):
    name, lq, lk, hq, hk, d, block_m, bnm, causal, mode, kind, blkk = case
    lk = lk or lq
    q, _, _, cuq = packed_inputs(lq, hq, hk, d, seed=seed, outliers=outliers)
    _, k, v, cuk = packed_inputs(lk, hq, hk, d, seed=seed + 1, outliers=outliers)
    return q, k, v, cuq, cuk, _bits(kind, lq, lk, hk, block_m, bnm, seed)


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_pipe_bitwise_equals_cpp_body(device, case):
    name = case[0]
    for seed, outliers in ((3, ()), (5, (7, 33, 70, 101))):
        inputs = _inputs(case, seed, tuple(c for c in outliers if c < case[5]))
        ref = _launch(device, inputs, case, pipe=False)
        got = _launch(device, inputs, case, pipe=True)
        same = got.view(np.uint16) == ref.view(np.uint16)
        print(f"pipe vs C++ body {name} seed {seed}: {same.mean():.6f} identical", flush=True)
        assert np.isfinite(got).all()
        assert same.all(), (name, seed, np.argwhere(~same)[:5])


@pytest.mark.parametrize("case", [c for c in CASES if c[0] in ("short_and_ragged", "lq_lt_lk", "blkk128",
                                                               "sptrans", "hd80_mha", "split_short_and_ragged",
                                                               "split_sptrans")],
                         ids=lambda c: c[0])
def test_pipe_matches_oracle(device, case):
    name, lq, lk, hq, hk, d, block_m, bnm, causal, mode, kind, blkk = case
    q, k, v, cuq, cuk, bits = _inputs(case, 9)
    got = _launch(device, (q, k, v, cuq, cuk, bits), case, pipe=True)
    q8, sq, cqs = O.quant_per_block_int8(q, cuq, 128)
    k8, sk, cks = O.quant_per_block_int8(k, cuk, blkk)
    ref = O.attn_fwd(q, k, v, cuq, cuk, bits, block_m=block_m, block_n_mask=bnm, causal=causal,
                     routing_mode={"mixed": 0, "fp16": 1, "int8": 2}[mode], q8=q8, k8=k8,
                     sq16=sq.astype(np.float16), sk16=sk.astype(np.float16), cu_q_scale=cqs, cu_k_scale=cks,
                     blkk=blkk)
    mx, mean = assert_close_out(got, ref)
    print(f"pipe vs oracle {name}: max-abs {mx:.3e} mean-abs {mean:.3e}", flush=True)


def _random_case(seed, split=False):
    """A seeded random launch of the pipelined instantiations: 1-4 ragged
    sequences (some shorter than a tile, some empty), GQA 1-4, head_dim
    65-128, block_m 128 or 256, causal or not, any routing mode and map
    (split: block_m 64 with mixed routing)."""
    rng = np.random.default_rng((2000 if split else 1000) + seed)
    nseq = int(rng.integers(1, 5))
    lq = [int(x) for x in rng.integers(0, 1100, size=nseq)]
    lq[int(rng.integers(0, nseq))] = int(rng.integers(300, 1100))
    causal = bool(rng.integers(0, 2))
    lk = None if causal or rng.integers(0, 2) == 0 else [int(x) for x in rng.integers(1, 1100, size=nseq)]
    if lk is not None:
        lk[int(np.argmax(lq))] = max(lk[int(np.argmax(lq))], max(lq))  # keep one max length for Q and K
    hk = int(rng.integers(1, 3))
    group = int(rng.choice([1, 2, 3, 4]))
    d = int(rng.choice([72, 96, 112, 128]))
    block_m = int(rng.choice([128, 128, 256]))
    bnm = int(rng.choice([64, 128]))
    mode = str(rng.choice(["mixed", "mixed", "fp16", "int8"]))
    blkk = int(rng.choice([64, 128]))
    if split:
        block_m, mode = 64, "mixed"
    return (f"random{'_split' if split else ''}{seed}", lq, lk, hk * group, hk, d, block_m, bnm, causal, mode,
            "rand", blkk)


@pytest.mark.parametrize("seed", range(8))
def test_pipe_random_launches_bitwise(device, seed):
    case = _random_case(seed)
    name = case[0]
    inputs = _inputs(case, 17 + seed)
    ref = _launch(device, inputs, case, pipe=False)
    got = _launch(device, inputs, case, pipe=True)
    same = got.view(np.uint16) == ref.view(np.uint16)
    print(f"pipe vs C++ body {case}: {same.mean():.6f} identical", flush=True)
    assert np.isfinite(got).all()
    assert same.all(), (name, np.argwhere(~same)[:5])


@pytest.mark.parametrize("seed", range(6))
def test_pipe_random_split_launches_bitwise(device, seed):
    case = _random_case(seed, split=True)
    name = case[0]
    inputs = _inputs(case, 41 + seed)
    ref = _launch(device, inputs, case, pipe=False)
    got = _launch(device, inputs, case, pipe=True)
    same = got.view(np.uint16) == ref.view(np.uint16)
    print(f"pipe vs C++ body {case}: {same.mean():.6f} identical", flush=True)
    assert np.isfinite(got).all()
    assert same.all(), (name, np.argwhere(~same)[:5])


@pytest.mark.parametrize("case", [c for c in CASES if c[0] in ("short_and_ragged", "split_short_and_ragged",
                                                               "long_causal_int8")],
                         ids=lambda c: c[0])
def test_group_interleave_keeps_outputs(device, case):
    """The work order (TILEMIX_HIP_INTERLEAVE: 1-4 groups of an XCD interleaved
    item by item) changes no output bit: every work item is computed once and
    on its own."""
    inputs = _inputs(case, 23)
    outs = []
    old = os.environ.get("TILEMIX_HIP_INTERLEAVE")
    try:
        for ilv in ("1", "2", "3", "4"):
            os.environ["TILEMIX_HIP_INTERLEAVE"] = ilv
            outs.append(_launch(device, inputs, case, pipe=True))
    finally:
        if old is None:
            os.environ.pop("TILEMIX_HIP_INTERLEAVE", None)
        else:
            os.environ["TILEMIX_HIP_INTERLEAVE"] = old
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint16), outs[0].view(np.uint16))
