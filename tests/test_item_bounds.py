"""The attention kernels' check of work items read from device memory
(work_item_fits, hexgen2_amd/csrc/hexkv_common.h), compiled for the host and
run on the CPU: in-range items pass; an item with any field outside the
call's geometry fails, including first/count values whose sum would overflow
int32 (such an item must not wrap into range and read past its row).  Needs
hipcc, not a GPU."""
import ctypes
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HIPCC = "/opt/rocm/bin/hipcc"
I32_MAX = 2**31 - 1

pytestmark = pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not installed")


@pytest.fixture(scope="module")
def fits(tmp_path_factory):
    out = tmp_path_factory.mktemp("items") / "libitems.so"
    cmd = [HIPCC, "-O1", "-fPIC", "-shared", "-std=c++17", "--offload-arch=gfx950", f"-I{ROOT / 'include'}",
           f"-I{ROOT / 'hexgen2_amd' / 'csrc'}", "-x", "hip", str(ROOT / "tests" / "emu" / "item_check.cpp"),
           "-o", str(out)]
    result = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert result.returncode == 0, result.stderr[-3000:]
    lib = ctypes.CDLL(str(out))
    lib.emu_item_fits.argtypes = [ctypes.c_int] * 11
    lib.emu_item_fits.restype = ctypes.c_int
    # geometry of the calls below: 8 rows, 4 head groups, 16 partitions, 5000 keys
    return lambda **kw: bool(lib.emu_item_fits(*[kw.get(k, v) for k, v in (
        ("row", 3), ("head_group", 1), ("part", 2), ("parts", 4), ("first", 2048), ("count", 1024),
        ("len", 4000), ("rows", 8), ("n_groups", 4), ("max_parts", 16), ("max_seqlen", 5000))]))


def test_in_range_items_pass(fits):
    assert fits()
    assert fits(first=0, count=4000)            # a whole row
    assert fits(first=3999, count=1)            # its last position
    assert fits(first=4000, count=0)            # an empty piece at the end
    assert fits(len=5000, first=4999, count=1)  # up to max_seqlen
    assert fits(row=7, head_group=3, part=15, parts=16)


@pytest.mark.parametrize("field,value", [
    ("row", 8), ("row", -1), ("head_group", 4), ("head_group", -1), ("part", 16), ("part", -1),
    ("parts", 0), ("parts", 17), ("first", -1), ("count", -1), ("len", 5001), ("count", 1953),
    ("first", 3001),
    # sums past int32: first + count would wrap negative and pass a naive check
    ("first", I32_MAX), ("count", I32_MAX),
])
def test_out_of_range_items_fail(fits, field, value):
    assert not fits(**{field: value})


def test_overflowing_sums_fail(fits):
    assert not fits(first=I32_MAX - 10, count=100, len=4000)
    assert not fits(first=100, count=I32_MAX - 50, len=4000)
    assert not fits(first=2**30, count=2**30 + 5, len=4000)
    assert not fits(first=-(2**31), count=2**31 - 1, len=4000)
