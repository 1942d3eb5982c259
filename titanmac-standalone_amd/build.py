"""Build libtmac.so, the C-ABI library of the TitanMAC sparse hot path, for gfx950.

Usage: python titanmac-standalone_amd/build.py [--jobs N]

Compiles every source under csrc/ with hipcc (cross-compiles without a GPU)
and links them into lib/libtmac.so next to this file. The library has no
torch dependency; Python loads it with ctypes after importing torch, whose
bundled HIP runtime (SONAME libamdhip64.so.7) then serves the library as well.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
OBJ_DIR = PKG_DIR / "_build"
LIB_DIR = PKG_DIR / "lib"
LIB_PATH = LIB_DIR / "libtmac.so"

ARCH = "gfx950"
# Packed-fp32 instructions are kept out of every kernel; hipcc's host pass
# warns that it does not know the feature, which is harmless.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
SOURCES = ["tmac_host.cpp", "bell_kernels.hip", "wattn_kernels.hip", "conv_kernels.hip",
           "norm_kernels.hip", "memory_kernels.hip"]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the gfx950 kernels need the ROCm toolchain")


def _compile(hipcc: str, src: Path, obj: Path) -> None:
    cmd = [hipcc, *HIP_FLAGS, "-x", "hip", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def build(jobs: int = 4, verbose: bool = True) -> Path:
    """Compile all sources and link lib/libtmac.so; returns the library path."""
    hipcc = _hipcc()
    OBJ_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    objs = [OBJ_DIR / (Path(s).stem + ".o") for s in SOURCES]
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        futs = [ex.submit(_compile, hipcc, CSRC / s, o) for s, o in zip(SOURCES, objs)]
        for f in futs:
            f.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--jobs", type=int, default=4)
    build(ap.parse_args().jobs)
