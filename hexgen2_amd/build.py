"""Compiles the hexkv HIP library (``libhexkv.so``) for gfx950, in tree.

``python -m hexgen2_amd.build`` rebuilds it; tests, ``bench.py`` and the
package load the built file and never compile by themselves.
"""
from __future__ import annotations

import concurrent.futures
import json
import os
import re
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
# Register, LDS and occupancy figures of the attention kernels, from the
# compiler's resource remarks: the work-list planner sizes row-block lists
# for the workgroups a CU holds at once (tests/test_kernel_resources.py).
RESOURCES = OBJDIR / "kernel_resources.json"
RESOURCE_SOURCES = {"hexkv_attend.hip"}


def _resources(remarks: str) -> dict:
    """{kernel symbol: {"vgprs", "agprs", "lds", "occupancy"}} from the
    -Rpass-analysis=kernel-resource-usage remarks of one compile."""
    out, name = {}, None
    fields = {"VGPRs": "vgprs", "AGPRs": "agprs", "LDS Size [bytes/block]": "lds",
              "Occupancy [waves/SIMD]": "occupancy"}
    for line in remarks.splitlines():
        m = re.search(r"remark: +Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            out[name] = {}
            continue
        m = re.search(r"remark: +([^:]+): (\d+)", line)
        if m and name and m.group(1).strip() in fields:
            out[name][fields[m.group(1).strip()]] = int(m.group(2))
    return out


def _compile(source: str):
    obj = OBJDIR / (source + ".o")
    cmd = [HIPCC, *COMMON, *DEVICE_FLAGS, "-x", "hip", "-c", str(CSRC / source), "-o", str(obj)]
    if source in RESOURCE_SOURCES:
        cmd.append("-Rpass-analysis=kernel-resource-usage")
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source}:\n{' '.join(cmd)}\n{result.stderr}")
    return obj, (_resources(result.stderr) if source in RESOURCE_SOURCES else {})


def build(verbose: bool = False) -> Path:
    """Compile every source and link ``libhexkv.so``; returns its path."""
    OBJDIR.mkdir(exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
        compiled = list(pool.map(_compile, SOURCES))
    objects = [obj for obj, _ in compiled]
    resources = {}
    for _, r in compiled:
        resources.update(r)
    RESOURCES.write_text(json.dumps(resources, indent=1, sort_keys=True) + "\n")
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
