"""Build libmhc_amd.so, the C-ABI library of the gfx950 mHC kernels.

Each csrc/*.hip file is compiled separately (in parallel) with hipcc for
gfx950 only, then linked into one shared object next to this file.  Packed
FP32 instructions are disabled for device code (-packed-fp32-ops), and so is
the accumulate-in-place dot2 encoding (-dot13-insts, see COMMON_FLAGS); hipcc's
host pass prints a harmless "not a recognized feature" warning for each.

Usage:  python minimind-mhc_amd/build.py [-v]
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libmhc_amd.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # v_dot2_f32_bf16 (VOP3P) instead of v_dot2c_f32_bf16: a product into a
    # zero accumulator is one instruction, not a v_mov of 0 plus the dot2c.
    "-Xclang", "-target-feature", "-Xclang", "-dot13-insts",
    "-Wall",
    "-Wno-unused-function",
    f"-I{REPO_DIR / 'include'}",
    f"-I{CSRC}",
]


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know these device feature names; drop that noise.
    noise = ("'-packed-fp32-ops' is not a recognized feature", "'-dot13-insts' is not a recognized feature")
    err = "\n".join(l for l in res.stderr.splitlines() if not any(n in l for n in noise))
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every kernel source and link libmhc_amd.so; returns its path."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = min(len(sources), max(1, min(16, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
