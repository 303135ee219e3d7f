"""Builds libturbo_decode_tail.so (HIP, gfx950) in-tree.

    python turbo-winfare_amd/build.py            # -> turbo-winfare_amd/lib/libturbo_decode_tail.so

Every source is compiled by hipcc for gfx950 only, with packed-FP32 instructions disabled, then
linked into one shared library that exports the C ABI of include/turbo_decode_tail.h.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "lib" / "libturbo_decode_tail.so"
SOURCES = ["api.cpp", "bundle.cpp", "prep.hip", "gemv_digits.hip", "gemm_mfma.hip", "select.hip", "misc.hip", "noalloc.hip", "matrix.cpp"]
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-fvisibility=hidden",
    # Fused multiply-add stays on by default, but `#pragma clang fp contract(off)` is honoured
    # where results must round like the reference's separate operations.
    "-ffp-contract=fast-honor-pragmas",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{PKG.parent / 'include'}",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    return str(cand) if cand.exists() else "hipcc"


# Per-source additions to FLAGS (later flags win).
SOURCE_FLAGS: dict[str, list[str]] = {}


def _compile(src: str) -> Path:
    out = OBJ / (Path(src).stem + ".o")
    cmd = [hipcc(), *FLAGS, *SOURCE_FLAGS.get(src, []), "-c", str(CSRC / src), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return out


def build(verbose: bool = False) -> Path:
    OBJ.mkdir(parents=True, exist_ok=True)
    LIB.parent.mkdir(parents=True, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", f"-Wl,-soname,{LIB.name}", "-o", str(tmp),
           *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
