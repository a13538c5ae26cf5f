"""Routing maps: bit-exact against vectors written by the reference's own
precision_maps.py (tests/golden/make_precision_map_goldens.py), plus
closed-form and invariant checks that need no reference."""
import json
import random
from pathlib import Path

import numpy as np
import pytest
import torch

from tilemix_amd.attention import precision_maps as pm

GOLDEN = json.loads((Path(__file__).parent / "golden" / "precision_maps_golden.json").read_text())


def _bits(entry):
    shape = entry["shape"]
    n = int(np.prod(shape))
    return np.unpackbits(np.frombuffer(bytes.fromhex(entry["bits"]), dtype=np.uint8))[:n].reshape(shape).astype(bool)


def _rows(packed):
    return [format(int(x), "016x") for x in packed.tolist()]


@pytest.mark.parametrize("case", GOLDEN["bitmask"], ids=lambda c: "{pattern_type}-L{seq_len}-m{BLOCK_M}-n{BLOCK_N}-p{percentage}".format(**c["kwargs"]))
def test_make_precision_bitmask_matches_reference(case):
    torch.manual_seed(case["torch_seed"])
    packed = pm.make_precision_bitmask(token_mask=None, **case["kwargs"])
    assert packed.dtype == torch.uint64
    assert _rows(packed) == case["rows"]


@pytest.mark.parametrize("entry", GOLDEN["token"], ids=lambda e: e["fn"])
def test_token_generators_and_token_path(entry):
    random.seed(entry["seed"])
    torch.manual_seed(entry["seed"])
    mask = getattr(pm, entry["fn"])(**entry["kwargs"])
    assert np.array_equal(mask[0, 0].numpy(), _bits(entry["mask"]))
    for label, pct, ptype in (("rows", None, "custom"), ("rows_pct", 0.6, "custom"),
                              ("rows_causal", None, "causal")):
        torch.manual_seed(11)
        packed = pm.make_precision_bitmask(
            seq_len=entry["kwargs"]["num_query"], BLOCK_M=64, BLOCK_N=64, token_mask=mask,
            percentage=pct, pattern_type=ptype, pattern_params=None, COMPUTE_BLOCK_N=64)
        assert _rows(packed) == entry[label], label


@pytest.mark.parametrize("entry", GOLDEN["weights"], ids=lambda e: str(e["args"]))
def test_causal_tile_weights(entry):
    w = pm._causal_compute_tile_weights(*entry["args"])
    assert w.dtype == torch.int64
    assert w.tolist() == entry["w"]


def test_causal_tile_weights_closed_form():
    # Sum of weights == number of causally executed 64-key tiles.
    for L, bm, bnm in [(4096, 128, 64), (32768, 128, 512), (1000, 64, 128)]:
        w = pm._causal_compute_tile_weights(L, bm, bnm, 64)
        nt = -(-L // 64)
        expected = sum(min(nt, -(-((r + 1) * bm) // 64)) for r in range(-(-L // bm)))
        assert int(w.sum()) == expected
    # cfg2: 32 query blocks x (2, 4, ..., 64) tiles = 1056
    assert int(pm._causal_compute_tile_weights(4096, 128, 64, 64).sum()) == 1056


def test_band_width_helper():
    for e in GOLDEN["band_width"]:
        assert pm.calculate_band_width_from_percentage(*e["args"]) == e["band_width"]


def test_block_layouts():
    g = GOLDEN["block"]
    layout = torch.tensor(g["layout"], dtype=torch.bool)
    assert np.array_equal(pm.gen_block_pattern(layout, g["block_size"])[0, 0].numpy(), _bits(g["block"]))
    assert np.array_equal(pm.layout_to_causal_mask(layout[None, None], g["block_size"])[0, 0].numpy(),
                          _bits(g["causal"]))


def _unpack(packed, ncol):
    v = np.array([int(x) for x in packed.tolist()], dtype=object)
    return np.array([[(int(r) >> j) & 1 for j in range(ncol)] for r in v], dtype=bool)


@pytest.mark.parametrize("p", [0.0, 0.25, 0.5, 0.75, 1.0])
def test_sptrans_cfg2_invariants(p):
    """SpTrans at the Llama-3.2-3B shape: INT8 bits only on legal groups and the
    weighted INT8 count is exactly round(1056 p) (all weights are 1 there)."""
    packed = pm.make_precision_bitmask(4096, 128, 64, None, percentage=p, pattern_type="sptrans",
                                       pattern_params={"stride": 128, "c": 32}, COMPUTE_BLOCK_N=64)
    bits = _unpack(packed, 64)
    w = pm._causal_compute_tile_weights(4096, 128, 64, 64).numpy()
    assert not (bits & (w == 0)).any()
    assert int((w * bits).sum()) == round(1056 * p)


def test_sptrans_pre_retarget_count():
    """Independent arithmetic: before retargeting, SpTrans marks 496 of the 1056
    legal cfg2 cells INT8 (so p=0.5 must add 32 cells)."""
    sparse = np.ones((32, 64), dtype=bool)
    for r in range(32):
        for key_stride in range(r + 1):  # stride 128 == block 128 -> one query stride per row
            pass
        sparse[r, 2 * r: 2 * r + 2] = False           # local stride (2 groups of 64)
        for s in range(r):                           # tail c=32 of earlier strides: group 2s+1
            sparse[r, 2 * s + 1] = False
    w = pm._causal_compute_tile_weights(4096, 128, 64, 64).numpy()
    assert int((sparse & (w > 0)).sum()) == 496


def test_zero_one_closed_form():
    for L, bm, bnm in [(256, 64, 64), (4096, 128, 64), (32768, 128, 512)]:
        z = pm.make_precision_bitmask(L, bm, bnm, None, pattern_type="zero", COMPUTE_BLOCK_N=64)
        o = pm.make_precision_bitmask(L, bm, bnm, None, pattern_type="one", COMPUTE_BLOCK_N=64)
        w = pm._causal_compute_tile_weights(L, bm, bnm, 64).numpy()
        assert all(int(x) == 0 for x in z.tolist())
        ones = [sum(1 << j for j in range(w.shape[1]) if w[r, j] > 0) for r in range(w.shape[0])]
        assert [int(x) for x in o.tolist()] == ones


def test_pack_is_lsb_first():
    m = torch.zeros((2, 64), dtype=torch.bool)
    m[0, 0] = True
    m[1, 63] = True
    assert [int(x) for x in pm.pack_block_precision_map(m).tolist()] == [1, 1 << 63]
    with pytest.raises(ValueError):
        pm.pack_block_precision_map(torch.zeros((2, 65), dtype=torch.bool))


def test_errors():
    with pytest.raises(ValueError):
        pm.make_precision_bitmask(4096, 128, 32, None, percentage=0.5, pattern_type="sptrans",
                                  pattern_params={})  # 128 groups > 64
    with pytest.raises(ValueError):
        pm.make_precision_bitmask(256, 64, 96, None, percentage=0.5, pattern_type="band",
                                  pattern_params={}, COMPUTE_BLOCK_N=64)
    with pytest.raises(ValueError):
        pm.make_precision_bitmask(256, 64, 64, None, percentage=None, pattern_type="band")
    with pytest.raises(ValueError):
        pm._retarget_weighted_int8_fraction(torch.zeros(2, 2, dtype=torch.bool),
                                            torch.ones(2, 2, dtype=torch.int64), 1.5)
    with pytest.raises(ValueError):
        pm._retarget_weighted_int8_fraction(torch.zeros(2, 2, dtype=torch.bool),
                                            torch.ones(2, 3, dtype=torch.int64), 0.5)


def test_row_rand_reseeds_global_rng():
    """Quirk kept: row_rand reseeds torch's global RNG with 42."""
    pm.make_precision_bitmask(4096, 128, 64, None, percentage=0.5, pattern_type="row_rand",
                              pattern_params={}, COMPUTE_BLOCK_N=64)
    after = torch.rand(3)
    torch.manual_seed(42)
    for _ in range(32):
        torch.randperm(64)
    assert torch.equal(after, torch.rand(3))
