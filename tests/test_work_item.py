"""The workgroup -> work-item mapping of the attention kernels (work_item in
tilemix_amd/csrc/attn_common.h), compiled for the host with hipcc and checked
on the CPU: every item is processed exactly once, a group of a whole round
stays on one XCD and is dispatched as one run of consecutive workgroups of
that XCD, its query blocks longest first."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module")
def dump_bin(tmp_path_factory):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("wi") / "work_item_dump"
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O1", "-std=c++17", f"-I{REPO / 'include'}",
                    f"-I{REPO / 'tilemix_amd' / 'csrc'}", str(REPO / "tests" / "native" / "work_item_dump.cpp"),
                    "-o", str(out)], check=True, capture_output=True)
    return out


def _mapping(dump_bin, groups, m_blocks, group):
    txt = subprocess.run([str(dump_bin), str(groups), str(m_blocks), str(group)], check=True,
                         capture_output=True, text=True).stdout
    return [tuple(int(v) for v in ln.split()) for ln in txt.splitlines()]


# (groups, m_blocks, group): cfg2 (B8 x Hk8, 32 blocks, GQA 3), the glue shape,
# cfg3 (4 groups: all dealt over the XCDs), cfg4-like, odd block counts, one
# block, a remainder of groups.
CASES = [(64, 32, 3), (64, 16, 3), (4, 256, 7), (192, 64, 4), (13, 5, 2), (16, 1, 3), (9, 7, 1), (8, 2, 8)]


@pytest.mark.parametrize("groups,m_blocks,group", CASES)
def test_work_item_mapping(dump_bin, groups, m_blocks, group):
    ipg = m_blocks * group
    total = groups * ipg
    pairs = _mapping(dump_bin, groups, m_blocks, group)
    items = [it for _, it in pairs if it >= 0]
    assert sorted(items) == list(range(total))
    rounds = groups // 8
    for x in range(8):
        seq = [it for bid, it in pairs if bid % 8 == x and it >= 0 and it // ipg < rounds * 8]
        # whole-round groups: x, x + 8, ...
        assert all((it // ipg) % 8 == x for it in seq)
        # group by group, each group's blocks longest first (mrev ascending)
        keyed = [(it // ipg, (it % ipg) // group) for it in seq]
        assert keyed == sorted(keyed)
