"""Resource figures the work-list planner relies on (no GPU needed).

The row-block chunk rule (hexgen2_amd/csrc/hexkv_attend.hip, rows_chunk)
sizes a list for the workgroups a CU holds at once: 4 of the kernel for 4
query heads per KV head (103 VGPRs, 33 KB of LDS), 5 of the others (84-96
VGPRs, 8-17 KB).  The build records the compiler's resource remarks for the
attention kernels; a kernel change that moves these counts must re-tune the
rule, and this test says so.
"""
import json
import re
from pathlib import Path

import pytest

RESOURCES = Path(__file__).resolve().parents[1] / "hexgen2_amd" / "_build" / "kernel_resources.json"
LDS_PER_CU = 160 * 1024


def row_block_kernels():
    if not RESOURCES.is_file():
        pytest.skip("the library has not been built here (python -m hexgen2_amd.build)")
    found = {}
    for name, r in json.loads(RESOURCES.read_text()).items():
        m = re.search(r"attend_rows_kernelIDF16[b_]Li128ELi(\d+)ELi(\d+)ELi(\d+)E", name)
        if m:
            found[name] = (int(m.group(1)), int(m.group(2)), r)
    assert found, "no row-block kernel in the resource record"
    return found


def test_row_block_workgroups_per_cu_match_the_planner():
    used = {(4, 2), (2, 2), (1, 2), (1, 4), (1, 8)}  # (query heads per KV head, head block) rows_block picks
    seen = set()
    for name, (gq, hb, r) in row_block_kernels().items():
        if (gq, hb) not in used:
            continue
        seen.add((gq, hb))
        want = 4 if gq == 4 else 5
        # one wave per SIMD per 256-thread workgroup: waves per SIMD = workgroups per CU
        held = min(r["occupancy"], LDS_PER_CU // r["lds"])
        assert held == want, f"{name}: {r} holds {held} workgroups per CU, the planner assumes {want}"
    assert seen == used


def test_resource_record_covers_every_attention_kernel():
    names = json.loads(RESOURCES.read_text()) if RESOURCES.is_file() else pytest.skip("not built")
    for kind in ("attend_valu_kernel", "attend_mfma_kernel", "attend_rows_kernel", "combine_kernel"):
        assert any(kind in n for n in names), kind
    for name, r in names.items():
        assert set(r) >= {"vgprs", "lds", "occupancy"}, name
