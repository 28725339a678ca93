"""Build recipe for libhynomas_fp8.so (gfx950), in-tree.

Compiles every ``csrc/*.hip`` with hipcc for gfx950 and links one shared
library next to this file. Runs on a machine without a GPU (hipcc
cross-compiles). Used by ``__graft_entry__.build()``.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB_NAME = "libhynomas_fp8.so"
LIB_PATH = PKG / LIB_NAME
OBJ_DIR = PKG / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    # Packed-FP32 instructions are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path) -> Path:
    OBJ_DIR.mkdir(exist_ok=True)
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile all HIP sources and link libhynomas_fp8.so; returns its path."""
    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources", file=sys.stderr)
    return LIB_PATH


STAMPS_LIB_PATH = PKG / "libhynomas_fp8_stamps.so"
STAMPS_SOURCE = "gemm_fp8.hip"


def build_stamps(verbose: bool = False) -> Path:
    """The measurement library libhynomas_fp8_stamps.so: the same objects as
    libhynomas_fp8.so with the GEMM compiled under HN_GEMM_PHASE_STAMPS (phase
    stamps of the persistent kernel, a workgroup cap from the environment),
    for ``bench.py --only gemm_phases``. Nothing in the product loads it.
    Call after build()."""
    OBJ_DIR.mkdir(exist_ok=True)
    src = CSRC / STAMPS_SOURCE
    obj = OBJ_DIR / "gemm_fp8_stamps.o"
    res = subprocess.run([HIPCC, *HIP_FLAGS, "-DHN_GEMM_PHASE_STAMPS", "-c", str(src), "-o", str(obj)],
                         capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name} (stamps):\n{res.stderr}")
    objs = [obj] + [OBJ_DIR / (p.stem + ".o") for p in sources() if p.name != STAMPS_SOURCE]
    tmp = STAMPS_LIB_PATH.with_suffix(".so.tmp")
    res = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)],
                         capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed (stamps):\n{res.stderr}")
    os.replace(tmp, STAMPS_LIB_PATH)
    if verbose:
        print(f"built {STAMPS_LIB_PATH}", file=sys.stderr)
    return STAMPS_LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    build_stamps(verbose=True)
