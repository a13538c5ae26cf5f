"""Build libtilemix_hip.so in-tree with hipcc for gfx950.

Usage: python -m tilemix_amd.csrc.build   (or tilemix_amd.csrc.build.build())

Every .hip file under this directory is compiled to an object in
tilemix_amd/_build/ (in parallel) and linked into tilemix_amd/libtilemix_hip.so.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG = CSRC.parent
REPO = PKG.parent
INCLUDE = REPO / "include"
BUILD_DIR = PKG / "_build"
LIB_NAME = "libtilemix_hip.so"
LIB_PATH = PKG / LIB_NAME

ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Bit-exact quantisation and score dequantisation rely on separately
    # rounded IEEE fp32 operations: no contraction into FMA, IEEE division.
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # Packed fp32 VALU forms are disabled for all device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mcode-object-version=5",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm at /opt/rocm)")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines()
        # hipcc's host pass does not know the device-only target feature.
        if "packed-fp32-ops" not in line and "not a recognized feature" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        sys.stderr.write(out + "\n")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every HIP source for gfx950 and link the shared library."""
    hipcc = _hipcc()
    # The pipelined tile loop's assembly is generated (attn_pipe_asm.h).
    sys.path.insert(0, str(CSRC))
    try:
        import gen_attn_pipe
    finally:
        sys.path.pop(0)
    gen_attn_pipe.write()
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    objs = [BUILD_DIR / (s.stem + ".o") for s in srcs]
    cmds = [[hipcc, *COMMON_FLAGS, "-c", str(s), "-o", str(o)] for s, o in zip(srcs, objs)]
    if verbose:
        for c in cmds:
            print(" ".join(c))
    jobs = jobs or min(len(cmds), max(1, (os.cpu_count() or 4)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(link))
    _run(link)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
