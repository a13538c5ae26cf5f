"""Write golden routing-map vectors from the reference's own precision_maps.py.

Run in the build container only (the reference is not present on GPU boxes and
is never shipped):

    python tests/golden/make_precision_map_goldens.py [/root/reference]

Why an import: the final routing maps of every percentage-driven layout go
through ``_retarget_weighted_int8_fraction`` (randperm under
``torch.Generator().manual_seed(42)``), ``row_rand`` / ``bigbird`` draw from the
global torch RNG and ``gen_row_rand_pattern`` from Python's ``random``; no
closed form pins those outputs, so their vectors come from the reference
function itself, on this container's torch.  Output:
tests/golden/precision_maps_golden.json (inputs + packed outputs, data only).
"""
from __future__ import annotations

import importlib.util
import json
import random
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
OUT = HERE / "precision_maps_golden.json"


def load_reference(root: Path):
    path = root / "attention" / "precision_maps.py"
    spec = importlib.util.spec_from_file_location("_reference_precision_maps", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def pick_mask_block_n(seqlen: int, compute_block_n: int) -> int:
    # models/tilemix_llama.py:46-49
    min_mask_bn = (seqlen + 63) // 64
    return ((max(min_mask_bn, compute_block_n) + compute_block_n - 1) // compute_block_n) * compute_block_n


def bits_hex(t: torch.Tensor) -> dict:
    a = t.detach().cpu().to(torch.bool).numpy()
    return {"shape": list(a.shape), "bits": np.packbits(a.reshape(-1)).tobytes().hex()}


def bitmask_cases():
    cases = []
    pcts = [0.0, 0.25, 0.5, 0.75, 1.0]
    # (seq_len, block_m, compute_block_n): block_n_mask from the model's rule.
    shapes = [(256, 64, 64), (1000, 64, 64), (4096, 128, 64), (8192, 128, 64), (32768, 128, 64)]
    params = {
        "band": {},
        "global": {"key_pos": [0, 1, 2, 3]},
        "row_rand": {},
        "align_sparse": {},
        "bigbird": {},
        "sptrans": {"stride": 128, "c": 32},
    }
    for seq_len, bm, bn in shapes:
        bnm = pick_mask_block_n(seq_len, bn)
        for pattern in ("zero", "one"):
            cases.append(dict(seq_len=seq_len, BLOCK_M=bm, BLOCK_N=bnm, COMPUTE_BLOCK_N=bn,
                              percentage=None, pattern_type=pattern, pattern_params={}))
        for pattern, pp in params.items():
            for p in pcts:
                if seq_len == 32768 and p not in (0.5,):
                    continue
                cases.append(dict(seq_len=seq_len, BLOCK_M=bm, BLOCK_N=bnm, COMPUTE_BLOCK_N=bn,
                                  percentage=p, pattern_type=pattern, pattern_params=pp))
    # SpTrans with default stride/c and odd lengths.
    for seq_len in (300, 2049, 5000):
        bnm = pick_mask_block_n(seq_len, 64)
        cases.append(dict(seq_len=seq_len, BLOCK_M=64, BLOCK_N=bnm, COMPUTE_BLOCK_N=64,
                          percentage=0.5, pattern_type="sptrans", pattern_params={}))
    # Mask groups of several compute tiles (MASK_GROUP > 1).
    for pattern in ("band", "sptrans", "bigbird", "row_rand", "align_sparse", "global"):
        cases.append(dict(seq_len=4096, BLOCK_M=128, BLOCK_N=256, COMPUTE_BLOCK_N=64,
                          percentage=0.5, pattern_type=pattern,
                          pattern_params={"stride": 128, "c": 32} if pattern == "sptrans" else {}))
    return cases


def main(root: Path) -> None:
    ref = load_reference(root)
    out = {"generator": "tests/golden/make_precision_map_goldens.py",
           "torch": torch.__version__, "bitmask": [], "token": [], "weights": []}

    for case in bitmask_cases():
        torch.manual_seed(1234)
        packed = ref.make_precision_bitmask(token_mask=None, **case)
        out["bitmask"].append({"kwargs": case, "torch_seed": 1234,
                               "rows": [format(int(x), "016x") for x in packed.tolist()]})

    # Token-mask path (percentage None, or a non-block policy with percentage):
    # masks from the reference generators under fixed seeds.
    token_specs = [
        ("gen_band_pattern", dict(num_query=300, num_key=300, band_width=None, percentage=0.5, block_n=64)),
        ("gen_band_pattern", dict(num_query=256, num_key=256, band_width=21)),
        ("gen_global_pattern", dict(num_query=200, num_key=200, key_pos=[0, 3, 150, 199, 250])),
        ("gen_row_rand_pattern", dict(num_query=96, num_key=128, num_rand_block_per_row=5)),
        ("gen_align_sparse_pattern", dict(num_query=300, num_key=300, alpha=32, beta=0.1)),
        ("gen_bigbird_pattern", dict(num_query=160, num_key=160, num_band_block=3, num_global_block=2,
                                     num_rand_block=3)),
        ("gen_causal_pattern", dict(num_query=130, num_key=130)),
    ]
    for fn, kw in token_specs:
        random.seed(7)
        torch.manual_seed(7)
        mask = getattr(ref, fn)(**kw)
        entry = {"fn": fn, "kwargs": kw, "seed": 7, "mask": bits_hex(mask[0, 0])}
        # The packed routing rows built from this token mask (no percentage,
        # and with the percentage-control flip under a fixed torch seed).
        for label, pct, ptype in (("rows", None, "custom"), ("rows_pct", 0.6, "custom"),
                                  ("rows_causal", None, "causal")):
            torch.manual_seed(11)
            packed = ref.make_precision_bitmask(
                seq_len=kw["num_query"], BLOCK_M=64, BLOCK_N=64, token_mask=mask,
                percentage=pct, pattern_type=ptype, pattern_params=None, COMPUTE_BLOCK_N=64)
            entry[label] = [format(int(x), "016x") for x in packed.tolist()]
        out["token"].append(entry)

    for seq_len, bm, bnm, bn in [(256, 64, 64, 64), (4096, 128, 64, 64), (32768, 128, 512, 64),
                                 (1000, 64, 128, 64), (8191, 128, 256, 64)]:
        w = ref._causal_compute_tile_weights(seq_len, bm, bnm, bn)
        out["weights"].append({"args": [seq_len, bm, bnm, bn], "w": w.tolist()})

    other = []
    for seq_len, pct, bn in [(4096, 0.5, 64), (4096, 0.3, None), (777, 0.8, 64), (100, 0.0, 64)]:
        other.append({"args": [seq_len, pct, bn],
                      "band_width": ref.calculate_band_width_from_percentage(seq_len, pct, bn)})
    out["band_width"] = other

    layout = torch.tensor([[1, 0, 1], [0, 1, 1], [1, 1, 0]], dtype=torch.bool)
    out["block"] = {"layout": layout.int().tolist(), "block_size": 4,
                    "block": bits_hex(ref.gen_block_pattern(layout, 4)[0, 0]),
                    "causal": bits_hex(ref.layout_to_causal_mask(layout[None, None], 4)[0, 0])}

    OUT.write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")
    print(f"wrote {OUT} ({len(out['bitmask'])} bitmask cases, {len(out['token'])} token cases)")


if __name__ == "__main__":
    main(Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/root/reference"))
