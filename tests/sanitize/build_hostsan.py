"""Build libtmac with AddressSanitizer + UndefinedBehaviorSanitizer on the HOST code.

Usage: python tests/sanitize/build_hostsan.py  ->  titanmac-standalone_amd/_build_hostsan/libtmac_hostsan.so

Every source is compiled with hipcc for gfx950 as in the product build, with each
sanitizer flag behind -Xarch_host, so only the host code (argument checks, the Block-ELL
index builders, the attention tile maps and work lists) is instrumented and the GPU
code objects are unchanged. The library leaves the sanitizer runtime symbols
undefined: a process that loads it must preload the runtime first, e.g.

  LD_PRELOAD=$(python tests/sanitize/build_hostsan.py --runtime) \\
  ASAN_OPTIONS=detect_leaks=0:halt_on_error=1 UBSAN_OPTIONS=halt_on_error=1:print_stacktrace=1 \\
  TMAC_LIB=titanmac-standalone_amd/_build_hostsan/libtmac_hostsan.so \\
  python -m pytest tests/test_host_abi.py -m "not gpu"

(tests/test_host_sanitizers.py runs exactly that.)
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import importlib.util
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
PKG = ROOT / "titanmac-standalone_amd"
OUT_DIR = PKG / "_build_hostsan"
LIB = OUT_DIR / "libtmac_hostsan.so"
SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
       "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer",
       "-Xarch_host", "-g"]


def _product_build():
    spec = importlib.util.spec_from_file_location("tmac_build", PKG / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def runtime() -> str:
    """Path of the clang ASan runtime (it carries the UBSan handlers too)."""
    hits = sorted(glob.glob("/opt/rocm/lib/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not hits:
        raise FileNotFoundError("libclang_rt.asan-x86_64.so not found under /opt/rocm/lib/llvm")
    return hits[-1]


def build() -> Path:
    b = _product_build()
    hipcc = b._hipcc()
    OUT_DIR.mkdir(exist_ok=True)
    objs = [OUT_DIR / (Path(s).stem + ".o") for s in b.SOURCES]

    def cc(src: str, obj: Path) -> None:
        cmd = [hipcc, *b.HIP_FLAGS, *SAN, "-x", "hip", "-c", str(b.CSRC / src), "-o", str(obj)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")

    with cf.ThreadPoolExecutor(max_workers=4) as ex:
        for f in [ex.submit(cc, s, o) for s, o in zip(b.SOURCES, objs)]:
            f.result()
    cmd = [hipcc, f"--offload-arch={b.ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(LIB)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    return LIB


if __name__ == "__main__":
    if "--runtime" in sys.argv:
        print(runtime())
    else:
        print(build())
