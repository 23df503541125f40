"""Compile the gfx950 HIP sources under kandle_amd/csrc into kandle_amd/libkandle_hip.so.

Usage: python -m kandle_amd.build   (or kandle_amd.build.build_library() from Python).

Each .hip file is compiled separately (in parallel) with hipcc for gfx950 only, then linked into one
shared library whose exported symbols are the C ABI declared in include/kandle_hip.h.  Packed fp32
instructions are disabled for all device code (-packed-fp32-ops).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libkandle_hip.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Per-source additions.  flash_prefill.hip is written NaN-free (masked scores are -inf, never NaN)
# and assumes no NaNs so that its row maxima compile to plain v_max3 without canonicalisation.
EXTRA_FLAGS = {"flash_prefill.hip": ["-fno-honor-nans"]}


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found: the HIP toolchain (ROCm) is required to build kandle_amd")
    return exe


def _compile(src: Path, obj: Path) -> None:
    cmd = [_hipcc(), *HIPCC_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless, filtered.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def build_library(verbose: bool = True) -> Path:
    """Compile every csrc/*.hip file for gfx950 and link libkandle_hip.so (always rebuilds)."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [BUILD_DIR / (s.stem + ".o") for s in sources]
    workers = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        futs = [ex.submit(_compile, s, o) for s, o in zip(sources, objs)]
        for f in futs:
            f.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} sources")
    return LIB_PATH


if __name__ == "__main__":
    build_library()
