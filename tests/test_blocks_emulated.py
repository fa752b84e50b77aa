"""The legacy-format kernels' index arithmetic, checked on the CPU.

tests/emu/blocks_emu.cpp compiles the real host code of hexkv_blocks.hip with
its kernel launches intercepted and replays every workgroup and lane on the
CPU, checking each access against the registered buffers.  The wrappers in
hexgen2_amd.kv_formats then run on host tensors through it, and every result
is compared with the oracle: the launch arguments the host code computes (tile
shapes, span folding, the wide and short-row launch shapes, the head gather's
shard columns, its per-layer and folded launches, its fallback to the span
engine) address exactly the right bytes and nothing outside the buffers.
Needs hipcc (it builds the emulator), not a GPU."""
import ctypes
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from hexgen2_amd import _lib
from hexgen2_amd import kv_formats as kvf
from oracle import kv_oracle as oracle

ROOT = Path(__file__).resolve().parents[1]
HIPCC = "/opt/rocm/bin/hipcc"
INT = {torch.float16: torch.int16, torch.bfloat16: torch.int16, torch.float32: torch.int32}

pytestmark = pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not installed")


@pytest.fixture(scope="module")
def emu(tmp_path_factory):
    out = tmp_path_factory.mktemp("emu") / "libemu.so"
    cmd = [HIPCC, "-O1", "-fPIC", "-shared", "-std=c++17", "--offload-arch=gfx950", f"-I{ROOT / 'include'}",
           f"-I{ROOT / 'hexgen2_amd' / 'csrc'}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-x", "hip", str(ROOT / "tests" / "emu" / "blocks_emu.cpp"),
           str(ROOT / "hexgen2_amd" / "csrc" / "hexkv_status.cpp"), "-o", str(out)]
    result = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert result.returncode == 0, result.stderr[-3000:]
    lib = ctypes.CDLL(str(out))
    vp, i64, ci = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    ptrs, blocks = ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(_lib.Block)
    lib.hexkv_flat_concat.argtypes = [blocks, ci, vp, vp]
    lib.hexkv_batch_pad.argtypes = [blocks, ci, ci, ptrs, i64, vp]
    lib.hexkv_head_concat.argtypes = [blocks, ci, ci, ptrs, vp]
    for f in (lib.hexkv_flat_concat, lib.hexkv_batch_pad, lib.hexkv_head_concat):
        f.restype = ci
    lib.hexkv_last_error.restype = ctypes.c_char_p
    lib.emu_register.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ci]
    lib.emu_violations.restype = ctypes.c_long
    lib.emu_launches.restype = ctypes.c_long
    return lib


@pytest.fixture
def run(emu, monkeypatch):
    """kv_formats bound to the emulator; outputs registered as destinations."""
    monkeypatch.setattr(kvf._lib, "load", lambda: emu)
    monkeypatch.setattr(kvf, "_require_device", lambda *t: None)
    monkeypatch.setattr(kvf, "_stream", lambda t: ctypes.c_void_p(0))
    real_empty = torch.empty

    def empty(*a, **k):
        k.pop("device", None)
        t = real_empty(*a, **k)
        emu.emu_register(t.untyped_storage().data_ptr(), t.untyped_storage().nbytes(), 1)
        return t
    monkeypatch.setattr(kvf.torch, "empty", empty)

    def sources(*tensors):
        emu.emu_clear()
        for t in tensors:
            if t.numel():
                emu.emu_register(t.untyped_storage().data_ptr(), t.untyped_storage().nbytes(), 0)
    return sources


def bits(t):
    return t.contiguous().view(INT[t.dtype]).numpy()


def rand(shape, dtype, seed):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed)).to(dtype)


def clean(emu, before):
    assert emu.emu_violations() == before, "an emulated access fell outside its buffers"


def test_flat_concat_cases(emu, run):
    big = rand((3, 4, 40, 2, 8, 16), torch.bfloat16, 1)
    stacked = rand((5, 1, 33, 2, 2, 16), torch.float32, 82)
    cases = [[big[l, :, :33] for l in range(3)],
             [rand((6, 5, 4), torch.float32, 2).permute(2, 0, 1)],
             [rand((3, 5, 7), torch.float16, 3), rand((2, 2), torch.float16, 4)],
             [rand((1, 4096, 2, 8, 16), torch.bfloat16, 5)],              # wide rows: 1024-thread launch
             [rand((1, 9, 2, 1, 16), torch.float32, 6 + i) for i in range(40)],  # two launches of spans
             [rand((0, 4), torch.float16, 7), rand((2, 4), torch.float16, 8)],
             [stacked[l, :, :30] for l in range(5)]]                      # layers folded
    v0 = emu.emu_violations()
    for ts in cases:
        run(*(ts + [big, stacked]))
        np.testing.assert_array_equal(bits(kvf.flat_concat(ts)), oracle.flat_concat([bits(t) for t in ts]))
    clean(emu, v0)


def test_batch_pad_cases(emu, run):
    v0 = emu.emu_violations()
    caches = rand((3, 5, 64, 2, 8, 16), torch.bfloat16, 3)
    dicts = [{l: caches[l, b0:b0 + b, :s] for l in range(3)}
             for b0, (b, s) in enumerate([(2, 61), (1, 7), (0, 5), (2, 0), (1, 64)])]
    run(caches)
    got = kvf.batch_key_value_memory_dicts(dicts)
    for l in range(3):
        np.testing.assert_array_equal(bits(got[l]), oracle.batch_pad([bits(d[l]) for d in dicts]))
    small = [{l: rand((b, s, 2, 1, 3), torch.float16, 100 * l + b) for l in range(20)}
             for b, s in ((1, 9), (2, 4), (1, 1))]
    run(*[t for d in small for t in d.values()])
    got = kvf.batch_key_value_memory_dicts(small, max_rows=16)           # 12-byte rows: 4-byte vectors
    for l in (0, 7, 19):
        np.testing.assert_array_equal(bits(got[l]), oracle.batch_pad([bits(d[l]) for d in small], max_rows=16))
    stack = rand((6, 2, 2048, 2, 4, 16), torch.float16, 80)               # wide rows, layers folded
    wide = [{l: stack[l, i:i + 1, :n] for l in range(6)} for i, n in enumerate((1931, 2048))]
    run(stack)
    got = kvf.batch_key_value_memory_dicts(wide)
    for l in (0, 5):
        np.testing.assert_array_equal(bits(got[l]), oracle.batch_pad([bits(d[l]) for d in wide]))
    clean(emu, v0)


def test_head_concat_gather_and_fallback(emu, run):
    v0 = emu.emu_violations()
    # one-head TP-8 shards, separate tensors per layer: one gather launch per
    # layer.  Each layer's shard is a view into its own buffer at an uneven
    # offset, so no two layers sit a fixed stride apart (which would let the
    # host fold them into one launch).
    base = [rand((4 * 300 * 2 * 128 + 64 * (l + 1) * (l + 2),), torch.bfloat16, 90 + l) for l in range(3)]
    shards = [{l: base[l][64 * (l + 1) * (l + 2) // 2:][:4 * 300 * 2 * 128].view(4, 300, 2, 1, 128)
               if j == 0 else rand((4, 300, 2, 1, 128), torch.bfloat16, 10 * j + l) for l in range(3)}
              for j in range(8)]
    run(*base)
    run(*[t for d in shards for t in d.values()])
    launches = emu.emu_launches()
    got = kvf.concat_dicts(shards)
    assert emu.emu_launches() - launches == 3
    for l in range(3):
        np.testing.assert_array_equal(bits(got[l]), oracle.concat_dim([bits(d[l]) for d in shards]))
    # shards of one stacked tensor: layers folded into one gather launch
    sh = rand((8, 4, 8, 64, 2, 1, 128), torch.bfloat16, 77)
    stacked = [{l: sh[j, l] for l in range(4)} for j in range(8)]
    run(sh)
    launches = emu.emu_launches()
    got = kvf.concat_dicts(stacked)
    assert emu.emu_launches() - launches == 1
    for l in (0, 3):
        np.testing.assert_array_equal(bits(got[l]), oracle.concat_dim([bits(d[l]) for d in stacked]))
    # strided, uneven and empty shards: the span engine
    bigh = rand((2, 3, 50, 2, 3, 64), torch.float16, 5)
    uneven = [{l: bigh[l, :, :41, :, :1] for l in range(2)}, {l: bigh[l, :, :41] for l in range(2)},
              {l: torch.zeros((3, 41, 2, 0, 64), dtype=torch.float16) for l in range(2)},
              {l: rand((3, 41, 2, 2, 64), torch.float16, 60 + l) for l in range(2)}]
    run(bigh, *[t for d in uneven for t in d.values()])
    got = kvf.concat_dicts(uneven)
    for l in range(2):
        np.testing.assert_array_equal(bits(got[l]), oracle.concat_dim([bits(d[l]) for d in uneven]))
    for dim in (-2, 1, 4, 0):
        shs = []
        for j, n in enumerate((2, 1, 3)):
            shape = [3, 5, 2, 2, 16]
            shape[dim % 5] = n
            shs.append({l: rand(tuple(shape), torch.float32, 7 * j + l) for l in range(2)})
        run(*[t for d in shs for t in d.values()])
        got = kvf.concat_dicts(shs, dim=dim)
        for l in range(2):
            np.testing.assert_array_equal(bits(got[l]), oracle.concat_dim([bits(d[l]) for d in shs], dim))
    clean(emu, v0)
