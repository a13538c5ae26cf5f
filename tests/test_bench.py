"""CPU checks of bench.py's accounting (no GPU): the algorithmic and
executed-tile op counts, the INT8 fraction of the SpTrans50 map and the
blended roofline times quoted for cfg2, and the single-GPU guard."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest

import bench

REPO = Path(__file__).resolve().parents[1]


def test_op_counts_cfg2():
    # 4 * B * Hq * D * L (L + 1) / 2 with the diagonal
    assert bench.algorithmic_ops() == pytest.approx(8.2484e11, rel=1e-4)
    # whole 128 x 64 tiles up to the diagonal: 1056 per (batch, head), 3.1% more
    assert bench.executed_tile_ops() == 4.0 * 8 * 24 * 128 * 128 * 64 * 1056
    assert bench.executed_tile_ops() / bench.algorithmic_ops() == pytest.approx(1.031, abs=1e-3)


def test_sptrans50_int8_fraction_and_roofline():
    import torch
    row, _ = bench.sptrans_map(0.5, torch.device("cpu"))
    f = bench.int8_fraction(row.tolist())
    assert f == 0.5  # target round(1056 * p) with unit weights
    ops = bench.algorithmic_ops()
    # roofline times quoted for cfg2: 0.3278 / 0.2868 / 0.2458 ms at f = 0 / 0.5 / 1
    for frac, ms in ((0.0, 0.3278), (0.5, 0.2868), (1.0, 0.2458)):
        assert bench.roofline_seconds(frac, ops) * 1e3 == pytest.approx(ms, abs=5e-5)


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120, cwd=REPO)
    assert r.returncode == 2
    assert "one MI355X" in r.stderr


def test_interleaved_timing_alternates():
    # Every function gets rounds x per samples, and the calls alternate
    # function by function in every round (no function timed all at once).
    calls = []

    def timer(f, n):
        calls.append((f, n))
        return [f] * n

    out = bench.interleaved(("a", "b", "c"), 5, 4, timer)
    assert calls == [(f, 4) for _ in range(5) for f in ("a", "b", "c")]
    assert out == [["a"] * 20, ["b"] * 20, ["c"] * 20]
