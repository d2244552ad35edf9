"""Build libqvex.so from csrc/*.hip with hipcc for gfx950.

Each translation unit is compiled separately (in parallel) and linked into one
shared library placed next to this file, so it travels with the source tree.

    python -m qvex.build            # from the qvex-3.5_amd directory
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT = PKG_DIR.parent                      # qvex-3.5_amd/
CSRC = ROOT / "csrc"
BUILD_DIR = ROOT / "_build"
LIB_PATH = PKG_DIR / "libqvex.so"
REPO = ROOT.parent
INCLUDE = REPO / "include"

ARCH = "gfx950"

# Packed-FP32 VALU ops stay off; contraction stays on except where a kernel's
# results must match a CPU emulation bit for bit. The first 16 dwords of every
# kernel's arguments are preloaded into SGPRs at wave launch (gfx950 kernarg
# preload; the code object keeps a loading prologue for firmware without it), so
# a wave issues its first loads without waiting for its argument loads: -1.1 %
# per decode cycle (2.081 -> 2.057 ms, same box, alternating libraries). MFMA
# accumulators stay in ordinary VGPRs (no v_accvgpr_read per use: 24 fewer VALU
# instructions per wave of the gate/up product; -3.6 us per cycle, 3 of 3 pairs).
COMMON_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wno-unused-command-line-argument", f"-I{INCLUDE}", f"-I{CSRC}",
]
PER_FILE_FLAGS = {
    "spec.hip": ["-ffp-contract=off"],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libqvex.so)")


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *PER_FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = True, jobs: int | None = None) -> Path:
    """Compile every csrc/*.hip and link libqvex.so; always rebuilds."""
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[qvex.build] {LIB_PATH} ({len(srcs)} units)", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build()
