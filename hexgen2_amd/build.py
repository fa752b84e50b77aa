"""Compiles the hexkv HIP library (``libhexkv.so``) for gfx950, in tree.

``python -m hexgen2_amd.build`` rebuilds it; tests, ``bench.py`` and the
package load the built file and never compile by themselves.
"""
from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
INCLUDE = ROOT / "include"
LIBRARY = PACKAGE / "libhexkv.so"
OBJDIR = PACKAGE / "_build"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# Packed-FP32 VALU forms are disabled for every device compile.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", f"-I{INCLUDE}", f"-I{CSRC}",
          "-Wall", "-Wno-unused-function"]
SOURCES = ["hexkv_status.cpp", "hexkv_copy.hip", "hexkv_attend.hip", "hexkv_blocks.hip", "hexkv_ipc.cpp"]


def _compile(source: str) -> Path:
    obj = OBJDIR / (source + ".o")
    cmd = [HIPCC, *COMMON, *DEVICE_FLAGS, "-x", "hip", "-c", str(CSRC / source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source}:\n{' '.join(cmd)}\n{result.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every source and link ``libhexkv.so``; returns its path."""
    OBJDIR.mkdir(exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
        objects = list(pool.map(_compile, SOURCES))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-o", str(tmp), *map(str, objects)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{result.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}", file=sys.stderr)
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
