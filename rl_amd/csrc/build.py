"""Build libmirl.so (gfx950) from the HIP/C++ sources in this directory.

Usage: ``python -m rl_amd.csrc.build`` or ``rl_amd.csrc.build.build()``.
The shared library is written next to the package (``rl_amd/libmirl.so``) so
that it travels with the source tree; object files go to ``csrc/_build``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG = HERE.parent
LIB_PATH = PKG / "libmirl.so"
BUILD_DIR = HERE / "_build"

SOURCES = [
    "host.cpp",
    "logprob.hip",
    "clipped_pg.hip",
    "advantage.hip",
    "topk_filter.hip",
    "topk_hist.hip",
    "topk_f32.hip",
    "linear_ce.hip",
    "divergence.hip",
    "packing.hip",
    "temperature.hip",
    "seq_errors.hip",
]

ARCH = "gfx950"

COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # packed FP32 VALU forms are kept out of generated code
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _compile(hipcc: str, src: str) -> Path:
    obj = BUILD_DIR / (Path(src).stem + ".o")
    cmd = [hipcc, *COMMON_FLAGS, "-c", str(HERE / src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(
        line
        for line in (proc.stderr or "").splitlines()
        if "packed-fp32-ops" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{errs}")
    if errs.strip():
        print(errs, file=sys.stderr)
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every source for gfx950 and link ``rl_amd/libmirl.so``."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(lambda s: _compile(hipcc, s), SOURCES))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
