"""A hazard the compiler does not pad inside inline assembly, checked on every
compiled kernel (CPU only: hipcc emits gfx950 assembly here).

A VALU instruction that writes an SGPR (v_readfirstlane, v_readlane reloading
a spilled SGPR, v_cmp with an SGPR destination) must be followed by 5 wait
states before a VMEM instruction reads that SGPR.  The compiler pads its own
VMEM instructions, but not those inside asm statements (the LDS-DMA copies of
the attention kernels and the pipelined loop's copies and scale loads): when
register pressure made the compiler reload a spilled buffer descriptor with
v_readlane right before a copy, the copy read a half-updated descriptor and
faulted.  The copy helper now pads 5 wait states; this test compiles every
source and scans the assembly in program order (across labels, which
over-approximates the paths) for a VMEM instruction inside an asm statement
that reads an SGPR written by VALU fewer than 5 wait states earlier.
"""
from __future__ import annotations

import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
CSRC = REPO / "tilemix_amd" / "csrc"

_SREG = re.compile(r"\bs\[(\d+):(\d+)\]|\bs(\d+)\b")


def _sregs(text: str) -> set[int]:
    out: set[int] = set()
    for m in _SREG.finditer(text):
        if m.group(1) is not None:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
        else:
            out.add(int(m.group(3)))
    return out


def scan(lines) -> list[tuple[str, str, int]]:
    """(function, instruction, wait states) of every violation."""
    fn, hits, recent, clock, in_asm = "?", [], [], 0, False
    for raw in lines:
        s = raw.strip()
        if re.match(r"^[A-Za-z_][A-Za-z0-9_]*:", s):
            fn, recent, clock = s.split(":")[0], [], 0
            continue
        if s.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if s.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if not s or s.startswith(";") or s.startswith("."):
            continue
        op = s.split()[0]
        ws = int(s.split()[1].rstrip(",")) + 1 if op == "s_nop" else 1
        if in_asm and op.startswith(("buffer_", "global_", "flat_", "scratch_")):
            reads = _sregs(s.split(None, 1)[1] if " " in s else "")
            for at, regs in recent:
                if regs & reads and clock - at - 1 < 5:
                    hits.append((fn, s, clock - at - 1))
        if op.startswith("v_") and not op.startswith("v_mfma") and " " in s:
            dst = s.split(None, 1)[1].split(",")[0].strip()
            if re.match(r"s(\d|\[)", dst):
                recent.append((clock, _sregs(dst)))
        clock += ws
        recent = [(at, r) for at, r in recent if clock - at <= 8]
    return hits


def test_scanner_catches_the_pattern():
    bad = ["k:", "v_readlane_b32 s47, v130, 25", ";;#ASMSTART", "s_nop 0",
           "buffer_load_dwordx4 v4, s[44:47], 0 offen lds", ";;#ASMEND"]
    assert scan(bad) and scan(bad)[0][2] == 1
    good = ["k:", "v_readlane_b32 s47, v130, 25", ";;#ASMSTART", "s_nop 4",
            "buffer_load_dwordx4 v4, s[44:47], 0 offen lds", ";;#ASMEND"]
    assert not scan(good)
    # the compiler's own loads (outside asm) are padded by the compiler
    assert not scan(["k:", "v_readfirstlane_b32 s4, v1", "buffer_load_dword v2, v3, s[4:7], 0 offen"])


@pytest.fixture(scope="module")
def device_asm(tmp_path_factory):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    sys_path = str(CSRC)
    import sys
    sys.path.insert(0, sys_path)
    try:
        import build as tb  # the flags of the real build
    finally:
        sys.path.pop(0)
    out = tmp_path_factory.mktemp("asm")

    def compile_one(src: Path) -> Path:
        dst = out / (src.stem + ".s")
        subprocess.run([hipcc, *tb.COMMON_FLAGS, "--cuda-device-only", "-S", str(src), "-o", str(dst)],
                       check=True, capture_output=True, cwd=str(CSRC))
        return dst

    with ThreadPoolExecutor(max_workers=8) as ex:
        return list(ex.map(compile_one, sorted(CSRC.glob("*.hip"))))


def test_no_sgpr_write_right_before_an_asm_vmem(device_asm):
    hits = []
    for path in device_asm:
        hits += [(path.name, *h) for h in scan(path.read_text().splitlines())]
    assert not hits, hits[:5]
