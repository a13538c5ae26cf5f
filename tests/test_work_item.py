"""The workgroup -> work-item mapping of the attention kernels (work_item in
tilemix_amd/csrc/attn_common.h), compiled for the host with hipcc and checked
on the CPU: every item is processed exactly once, a group of a whole round
stays on one XCD, the XCD's groups run `ilv` at a time interleaved item by
item, each group's query blocks longest first; and the interleave chosen per
launch (interleave_groups) keeps the interleaved groups' K/V near one L2."""
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


def _mapping(dump_bin, groups, m_blocks, group, ilv):
    txt = subprocess.run([str(dump_bin), str(groups), str(m_blocks), str(group), str(ilv)], check=True,
                         capture_output=True, text=True).stdout
    return [tuple(int(v) for v in ln.split()) for ln in txt.splitlines()]


# (groups, m_blocks, group): cfg2 (B8 x Hk8, 32 blocks, GQA 3), the glue shape,
# cfg3 (4 groups: all dealt over the XCDs), cfg4-like, odd block counts, one
# block, a remainder of groups.
CASES = [(64, 32, 3), (64, 16, 3), (4, 256, 7), (192, 64, 4), (13, 5, 2), (16, 1, 3), (9, 7, 1), (8, 2, 8)]


@pytest.mark.parametrize("ilv", [1, 2, 3, 4])
@pytest.mark.parametrize("groups,m_blocks,group", CASES)
def test_work_item_mapping(dump_bin, groups, m_blocks, group, ilv):
    ipg = m_blocks * group
    total = groups * ipg
    pairs = _mapping(dump_bin, groups, m_blocks, group, ilv)
    items = [it for _, it in pairs if it >= 0]
    assert sorted(items) == list(range(total))
    rounds = groups // 8
    for x in range(8):
        seq = [it for bid, it in pairs if bid % 8 == x and it >= 0 and it // ipg < rounds * 8]
        # whole-round groups: x, x + 8, ...
        assert all((it // ipg) % 8 == x for it in seq)
        # chunks of ilv groups (their rank on the XCD: (it // ipg) // 8), the
        # chunk's groups taking turns item by item, each group's items in order
        # (query blocks longest first, mrev ascending)
        rank = [(it // ipg) // 8 for it in seq]
        assert [r // ilv for r in rank] == sorted(r // ilv for r in rank)
        for c in range(0, rounds, ilv):
            kc = min(ilv, rounds - c)
            chunk = [(r, it % ipg) for r, it in zip(rank, seq) if c <= r < c + kc]
            assert len(chunk) == kc * ipg
            assert [r for r, _ in chunk] == [c + w % kc for w in range(kc * ipg)]
            assert [i for _, i in chunk] == [w // kc for w in range(kc * ipg)]


@pytest.mark.parametrize("max_seqlen_k,head_dim,expected", [
    (4096, 128, 2), (2048, 128, 4), (8192, 128, 1), (1024, 128, 4), (32768, 128, 1), (4096, 64, 4),
    (6000, 128, 1), (3000, 128, 3), (0, 128, 4)])
def test_interleave_choice(dump_bin, max_seqlen_k, head_dim, expected):
    """Groups interleaved per XCD: as many as keep fp16 K, V and int8 K of the
    groups within ~5.5 MB (a little over one 4 MB L2), 1 to 4."""
    out = subprocess.run([str(dump_bin), "--ilv", str(max_seqlen_k), str(head_dim)], check=True,
                         capture_output=True, text=True).stdout
    assert int(out) == expected
    assert max_seqlen_k * head_dim * 5 * expected <= 5632 * 1024 or expected == 1
