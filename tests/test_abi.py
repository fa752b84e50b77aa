"""The C-ABI boundary, checked without a GPU: the built library loads, exports
every function include/hexkv.h declares, the ctypes mirror of
``hexkv_attend_params`` has the C layout, and argument validation fails
before any launch."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest
import torch

from hexgen2_amd import _lib, ops

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "hexkv.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(hexkv_[a-z_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared_functions() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.hexkv_version() >= 100
    # a successful call clears the thread's last error
    p = _lib.AttendParams(q_heads=8, kv_heads=2, kernel=0)
    assert lib.hexkv_attend_kernel(ctypes.byref(p)) == 1
    assert lib.hexkv_last_error() == b""


@pytest.mark.parametrize("c_name,mirror", [("hexkv_attend_params", _lib.AttendParams),
                                            ("hexkv_ft_attend_params", _lib.FtAttendParams),
                                            ("hexkv_block", _lib.Block),
                                            ("hexkv_ipc_handle", _lib.IpcHandle),
                                            ("hexkv_work_item", _lib.WorkItem)])
def test_struct_layouts_match_c(tmp_path, c_name, mirror):
    fields = [f[0] for f in mirror._fields_]
    src = tmp_path / "layout.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "hexkv.h"\nint main(void){\n'
                   f'printf("%zu\\n", sizeof({c_name}));\n'
                   + "".join(f'printf("%zu\\n", offsetof({c_name}, {f}));\n' for f in fields)
                   + "return 0;}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)],
                   check=True)
    values = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert values[0] == ctypes.sizeof(mirror)
    assert values[1:] == [getattr(mirror, f).offset for f in fields]


def test_header_compiles_as_cxx(tmp_path):
    src = tmp_path / "x.cpp"
    src.write_text('#include "hexkv.h"\nint (*volatile probe)(void) = &hexkv_version;\nint main(){ return probe == nullptr; }\n')
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Werror", "-c", f"-I{ROOT / 'include'}", str(src),
                    "-o", str(tmp_path / "x.o")], check=True)


def test_validation_fails_before_launch():
    lib = _lib.load()
    ptr = (ctypes.c_void_p * 1)(16)
    lens = (ctypes.c_int64 * 1)(9)
    # length above capacity -> HEXKV_ERANGE, nothing launched
    assert lib.hexkv_pack(ptr, ptr, 1, 1, 8, 8, 512, lens, None) == _lib.HEXKV_ERANGE
    assert b"outside" in lib.hexkv_last_error()
    assert lib.hexkv_pack(ptr, ptr, 1, 1, 8, 8, 510, lens, None) == _lib.HEXKV_EINVAL
    assert lib.hexkv_append(None, None, 1, 8, 8, 512, None, 0, None) == _lib.HEXKV_EINVAL
    assert lib.hexkv_append(16, 16, 1, 8, 8, 512, None, 8, None) == _lib.HEXKV_ERANGE
    p = _lib.AttendParams(dtype=1, batch=1, q_len=1, q_heads=4, kv_heads=2, head_dim=48, capacity=8, max_seqlen=4)
    assert lib.hexkv_attend(ctypes.byref(p), None, 0, None) == _lib.HEXKV_EUNSUPPORTED
    p.head_dim, p.q_heads = 64, 3
    assert lib.hexkv_attend(ctypes.byref(p), None, 0, None) == _lib.HEXKV_EINVAL
    p.q_heads, p.max_seqlen = 4, 9
    assert lib.hexkv_attend(ctypes.byref(p), None, 0, None) == _lib.HEXKV_ERANGE
    # nothing to do is not an error
    assert lib.hexkv_pack(ptr, ptr, 0, 1, 8, 8, 512, lens, None) == _lib.HEXKV_OK


def test_legacy_format_validation_fails_before_launch():
    lib = _lib.load()
    B = _lib.Block
    ptr = (ctypes.c_void_p * 2)(16, 32)
    # negative size, missing data pointer, missing destination
    assert lib.hexkv_flat_concat((B * 1)(B(16, -1, 1, 1, 0, 0)), 1, 64, None) == _lib.HEXKV_EINVAL
    assert lib.hexkv_flat_concat((B * 1)(B(None, 8, 1, 1, 8, 8)), 1, 64, None) == _lib.HEXKV_EINVAL
    assert lib.hexkv_flat_concat((B * 1)(B(16, 8, 1, 1, 8, 8)), 1, None, None) == _lib.HEXKV_EINVAL
    # empty blocks move nothing
    assert lib.hexkv_flat_concat((B * 1)(B(None, 8, 0, 1, 8, 8)), 1, None, None) == _lib.HEXKV_OK
    # a request longer than max_rows; widths or sizes that differ over layers
    two = (B * 2)(B(16, 512, 5, 1, 512, 2560), B(32, 512, 5, 1, 512, 2560))
    assert lib.hexkv_batch_pad(two, 2, 1, ptr, 4, None) == _lib.HEXKV_ERANGE
    assert b"max_rows" in lib.hexkv_last_error()
    two[1].height = 4
    assert lib.hexkv_batch_pad(two, 2, 1, ptr, 8, None) == _lib.HEXKV_EINVAL
    two[1].height, two[1].width = 5, 256
    assert lib.hexkv_batch_pad(two, 2, 1, ptr, 8, None) == _lib.HEXKV_EINVAL
    # shards of one layer with different heights; a shard width that changes over layers
    shards = (B * 2)(B(16, 256, 6, 2, 256, 1536), B(32, 256, 5, 2, 256, 1280))
    assert lib.hexkv_head_concat(shards, 1, 2, ptr, None) == _lib.HEXKV_EINVAL
    shards[1].height, shards[1].width = 6, 512
    assert lib.hexkv_head_concat(shards, 2, 1, ptr, None) == _lib.HEXKV_EINVAL


def test_ft_validation_fails_before_launch():
    lib = _lib.load()
    P = _lib.FtAttendParams
    base = dict(dtype=1, batch=1, q_heads=4, kv_heads=2, head_dim=64, softmax_scale=0.125, capacity=8,
                max_position=3, q=16, k_new=16, v_new=16, k_cache=16, v_cache=16, out=16)
    assert lib.hexkv_ft_attend(ctypes.byref(P(**{**base, "max_position": 8})), None, 0, None) == _lib.HEXKV_ERANGE
    assert lib.hexkv_ft_attend(ctypes.byref(P(**{**base, "rotary_dim": 3})), None, 0, None) == _lib.HEXKV_EINVAL
    assert lib.hexkv_ft_attend(ctypes.byref(P(**{**base, "rotary_dim": 66})), None, 0, None) == _lib.HEXKV_EINVAL
    assert lib.hexkv_ft_attend(ctypes.byref(P(**{**base, "rotary_dim": 64})), None, 0, None) == _lib.HEXKV_EINVAL
    assert b"rotary_base" in lib.hexkv_last_error()
    assert lib.hexkv_ft_attend(ctypes.byref(P(**{**base, "head_dim": 48})), None, 0, None) == _lib.HEXKV_EUNSUPPORTED
    assert lib.hexkv_ft_attend(ctypes.byref(P(**{**base, "q_heads": 3})), None, 0, None) == _lib.HEXKV_EINVAL
    assert lib.hexkv_ft_attend(ctypes.byref(P(**{**base, "out": 0})), None, 0, None) == _lib.HEXKV_EINVAL
    assert lib.hexkv_ft_attend(ctypes.byref(P(**{**base, "batch": 0})), None, 0, None) == _lib.HEXKV_OK
    # ft_store: more positions than capacity; a head_dim that is not whole 16-byte chunks
    assert lib.hexkv_ft_store(16, 0, 0, 0, 16, 16, 1, 9, 8, 2, 64, 1, None) == _lib.HEXKV_ERANGE
    assert lib.hexkv_ft_store(16, 0, 0, 0, 16, 16, 1, 4, 8, 2, 12, 1, None) == _lib.HEXKV_EINVAL
    assert lib.hexkv_ft_store(None, 0, 0, 0, 16, 16, 1, 0, 8, 2, 64, 1, None) == _lib.HEXKV_OK


def test_status_codes_map_to_reference_exception_types():
    with pytest.raises(ValueError):
        _lib.check(_lib.HEXKV_EINVAL, "x")
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.HEXKV_EUNSUPPORTED, "x")
    with pytest.raises(_lib.HexKVError):
        _lib.check(_lib.HEXKV_EHIP, "x")


def test_cpu_tensors_are_rejected_loudly():
    cache = torch.zeros((1, 4, 2, 1, 8))
    with pytest.raises(ValueError, match="no CPU fallback"):
        ops.pack_live([cache], [2])
    with pytest.raises(ValueError, match="no CPU fallback"):
        ops.decode_attention(torch.zeros((1, 1, 2, 8)), cache, max_seqlen=2, seqlen_bias=2)


@pytest.mark.parametrize("hq,hkv,d,dtype,kernel,expect", [
    (32, 8, 128, torch.bfloat16, "auto", "valu"),    # Llama-3-8B: group 4
    (8, 1, 128, torch.bfloat16, "auto", "mfma"),     # Llama-2-70B TP-8 share: group 8
    (32, 4, 64, torch.float16, "auto", "mfma"),      # TinyLlama: group 8, head_dim 64
    (32, 32, 128, torch.float16, "auto", "valu"),    # Llama-2-7B: group 1
    (8, 1, 128, torch.float32, "auto", "valu"),      # fp32 never takes the matrix cores
    (8, 1, 32, torch.float16, "auto", "valu"),       # head_dim below 64
    (8, 1, 128, torch.bfloat16, "valu", "valu"),
    (32, 8, 128, torch.bfloat16, "mfma", "mfma"),
    (32, 8, 128, torch.bfloat16, "rows", "rows")])
def test_attend_kernel_choice(hq, hkv, d, dtype, kernel, expect):
    """hexkv_attend_kernel resolves the kernel choice from geometry alone
    (no device memory is touched)."""
    q = torch.empty((2, 1, hq, d), dtype=dtype)
    cache = torch.empty((2, 16, 2, hkv, d), dtype=dtype)
    assert ops.attend_kernel(q, cache, kernel) == expect


def test_attend_kernel_rejects_bad_geometry():
    p = _lib.AttendParams()
    p.q_heads, p.kv_heads = 6, 4
    assert _lib.load().hexkv_attend_kernel(ctypes.byref(p)) == _lib.HEXKV_EINVAL
    assert b"q_heads" in _lib.load().hexkv_last_error()


def test_noalloc_scratch_limit_matches_header_and_rejects_oversized_calls(tmp_path):
    src = tmp_path / "limit.c"
    src.write_text('#include <stdio.h>\n#include "hexkv.h"\n'
                   'int main(void){ printf("%u\\n", HEXKV_NOALLOC_SCRATCH_BYTES); return 0; }\n')
    exe = tmp_path / "limit"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)],
                   check=True)
    limit = int(subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout)
    assert limit == _lib.NOALLOC_SCRATCH_BYTES
    # A request whose split-K partials exceed the static scratch is refused on
    # the host, before any HIP call: 4096 rows x 32 heads x 64 partitions.
    lib = _lib.load()
    p = _lib.AttendParams(dtype=_lib.HEXKV_BF16, batch=4096, q_len=1, q_heads=32, kv_heads=8, head_dim=128,
                          softmax_scale=0.088, q=0x10000, q_batch_stride=32 * 128, q_row_stride=32 * 128,
                          cache=0x20000, cache_batch_stride=8192 * 2048, cache_pos_stride=2048,
                          cache_kv_stride=1024, capacity=8192, out=0x30000, out_batch_stride=32 * 128,
                          out_row_stride=32 * 128, seqlen_bias=8192, max_seqlen=8192, partition=128)
    need = lib.hexkv_attend_workspace_bytes(ctypes.byref(p))
    assert need > limit
    assert lib.hexkv_attend_noalloc(ctypes.byref(p), None) == _lib.HEXKV_EWORKSPACE
    assert b"static scratch" in lib.hexkv_last_error()


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    """Without the built library every entry point raises (there is no CPU
    path to fall back to): the loader names the missing file."""
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIBRARY", tmp_path / "libhexkv.so")
    with pytest.raises(RuntimeError, match="missing"):
        _lib.load()
    with pytest.raises(RuntimeError, match="missing"):
        ops.attend_kernel(torch.zeros((1, 1, 8, 64), dtype=torch.float16),
                          torch.zeros((1, 4, 2, 1, 64), dtype=torch.float16))


def test_empty_batch_with_a_work_list_launches_nothing():
    """An empty batch plans an empty list and the call returns HEXKV_OK
    without launching, with or without a work list (no GPU needed: nothing
    reaches the runtime)."""
    lib = _lib.load()
    p = _lib.AttendParams(dtype=1, batch=0, q_len=1, q_heads=8, kv_heads=2, head_dim=64, capacity=8,
                          max_seqlen=4, softmax_scale=0.125)
    n, mp = ctypes.c_int32(), ctypes.c_int32()
    lens = (ctypes.c_int32 * 1)()
    assert lib.hexkv_attend_plan(ctypes.byref(p), lens, None, 0, None, 0, ctypes.byref(n), ctypes.byref(mp)) == 0
    assert n.value == 0
    assert lib.hexkv_attend(ctypes.byref(p), None, 0, None) == _lib.HEXKV_OK
    p.work_items_dev, p.work_parts_dev, p.n_work_items, p.work_max_parts, p.work_xcds = 256, 256, 0, 1, 8
    assert lib.hexkv_attend(ctypes.byref(p), None, 0, None) == _lib.HEXKV_OK
    assert lib.hexkv_last_error() == b""


def test_single_launch_and_lengths_out_validation():
    """work_xcds and lengths_out_dev are checked before any launch."""
    lib = _lib.load()
    p = _lib.AttendParams(dtype=1, batch=1, q_len=1, q_heads=8, kv_heads=2, head_dim=64, capacity=8,
                          max_seqlen=4, softmax_scale=0.125, q=256, cache=256, out=256,
                          cache_batch_stride=8 * 2 * 2 * 64, cache_pos_stride=2 * 2 * 64, cache_kv_stride=128)
    p.work_xcds = 8  # without a work list
    assert lib.hexkv_attend(ctypes.byref(p), None, 0, None) == _lib.HEXKV_EINVAL
    assert b"work lists" in lib.hexkv_last_error()
    p.work_xcds = 65
    assert lib.hexkv_attend(ctypes.byref(p), None, 0, None) == _lib.HEXKV_EINVAL
    p.work_xcds, p.lengths_out_dev = 0, 256  # lengths_out without a work list and kv_new
    assert lib.hexkv_attend(ctypes.byref(p), None, 0, None) == _lib.HEXKV_EINVAL
    assert b"lengths_out_dev" in lib.hexkv_last_error()
    assert lib.hexkv_device_status(None, 0, None) == _lib.HEXKV_EINVAL
    assert lib.hexkv_device_xcds(None) == _lib.HEXKV_EINVAL


def test_row_block_kernel_validation():
    """HEXKV_KERNEL_ROWS is refused before any launch outside what it runs:
    work lists planned for 1-8 XCDs with at most 64 partitions per segment,
    16-bit data, head_dim 128, 2+ KV heads and 1, 2 or 4 query heads each."""
    lib = _lib.load()

    def params(**kw):
        g = dict(dtype=1, batch=1, q_len=1, q_heads=32, kv_heads=8, head_dim=128, capacity=8, max_seqlen=4,
                 softmax_scale=0.125, q=256, cache=256, out=256, cache_batch_stride=8 * 2 * 8 * 128,
                 cache_pos_stride=2 * 8 * 128, cache_kv_stride=8 * 128, kernel=3, work_items_dev=256,
                 work_parts_dev=256, n_work_items=1, work_max_parts=2, work_xcds=8)
        g.update(kw)
        return _lib.AttendParams(**g)

    for kw in (dict(work_items_dev=None, work_parts_dev=None, work_xcds=0),  # grid mode
               dict(work_xcds=0),                                           # not planned for the XCDs
               dict(work_max_parts=65),                                     # more pieces than the merge takes
               dict(dtype=2, cache_batch_stride=8 * 2 * 8 * 128),           # fp32
               dict(head_dim=64, cache_batch_stride=8 * 2 * 8 * 64, cache_pos_stride=2 * 8 * 64,
                    cache_kv_stride=8 * 64),                                # head_dim 64
               dict(q_heads=8, kv_heads=1, cache_batch_stride=8 * 2 * 128, cache_pos_stride=2 * 128,
                    cache_kv_stride=128),                                   # one KV head
               dict(q_heads=64)):                                           # group 8
        assert lib.hexkv_attend(ctypes.byref(params(**kw)), None, 0, None) == _lib.HEXKV_EUNSUPPORTED, kw
    p = params(kernel=4)
    assert lib.hexkv_attend(ctypes.byref(p), None, 0, None) == _lib.HEXKV_EINVAL
    assert lib.hexkv_attend_kernel(ctypes.byref(params())) == _lib.KERNELS["rows"]
