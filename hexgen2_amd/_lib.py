"""ctypes binding of ``libhexkv.so`` (the C ABI declared in ``include/hexkv.h``).

The library is built in tree by ``python -m hexgen2_amd.build``.  Loading it
fails loudly when it is missing: there is no CPU fallback for the data path.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIBRARY = Path(__file__).resolve().parent / "libhexkv.so"

HEXKV_F16, HEXKV_BF16, HEXKV_F32 = 0, 1, 2
KERNELS = {"auto": 0, "valu": 1, "mfma": 2, "rows": 3}
HEXKV_OK = 0
HEXKV_EINVAL, HEXKV_ERANGE, HEXKV_EHIP, HEXKV_EUNSUPPORTED, HEXKV_EWORKSPACE = -1, -2, -3, -4, -5
MAX_LAYERS_PER_LAUNCH = 96
MAX_SEQS_PER_LAUNCH = 256

# Every symbol the header declares; tests check the library exports them all.
EXPORTS = ("hexkv_version", "hexkv_last_error", "hexkv_pack", "hexkv_unpack", "hexkv_append",
           "hexkv_attend_workspace_bytes", "hexkv_attend_kernel", "hexkv_attend", "hexkv_flat_concat", "hexkv_batch_pad",
           "hexkv_head_concat", "hexkv_ipc_export", "hexkv_ipc_open", "hexkv_ipc_close",
           "hexkv_ipc_dlpack", "hexkv_ft_store", "hexkv_ft_attend_workspace_bytes", "hexkv_ft_attend",
           "hexkv_attend_noalloc", "hexkv_attend_plan", "hexkv_attend_plan_chunk", "hexkv_attend_plan_kernel",
           "hexkv_device_status", "hexkv_device_xcds")
NOALLOC_SCRATCH_BYTES = 32 << 20
# Arrival counters at the front of every attention workspace (zero them once).
ATTEND_COUNTER_BYTES = 256 << 10
ATTEND_COUNTER_WORDS = ATTEND_COUNTER_BYTES // 8  # one 64-bit counter per (row, head group)
# Device status flags (hexkv_device_status).
STATUS_APPEND_SKIPPED, STATUS_LENGTH_CLAMPED, STATUS_PLACEMENT, STATUS_DISPATCH, STATUS_LIST = 1, 2, 4, 8, 16
STATUS_ERRORS = STATUS_APPEND_SKIPPED | STATUS_LENGTH_CLAMPED | STATUS_PLACEMENT | STATUS_LIST


class AttendParams(ctypes.Structure):
    """Mirror of ``hexkv_attend_params``."""
    _fields_ = [
        ("dtype", ctypes.c_int), ("batch", ctypes.c_int), ("q_len", ctypes.c_int),
        ("q_heads", ctypes.c_int), ("kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int),
        ("causal", ctypes.c_int), ("softmax_scale", ctypes.c_float),
        ("q", ctypes.c_void_p), ("q_batch_stride", ctypes.c_int64), ("q_row_stride", ctypes.c_int64),
        ("cache", ctypes.c_void_p), ("cache_batch_stride", ctypes.c_int64),
        ("cache_pos_stride", ctypes.c_int64), ("cache_kv_stride", ctypes.c_int64),
        ("capacity", ctypes.c_int64),
        ("out", ctypes.c_void_p), ("out_batch_stride", ctypes.c_int64), ("out_row_stride", ctypes.c_int64),
        ("seqlens_dev", ctypes.c_void_p), ("seqlen_bias", ctypes.c_int32), ("max_seqlen", ctypes.c_int32),
        ("kv_new", ctypes.c_void_p), ("partition", ctypes.c_int), ("kernel", ctypes.c_int),
        ("work_items_dev", ctypes.c_void_p), ("work_parts_dev", ctypes.c_void_p),
        ("n_work_items", ctypes.c_int32), ("work_max_parts", ctypes.c_int32),
        ("work_xcds", ctypes.c_int32), ("lengths_out_dev", ctypes.c_void_p),
    ]


class WorkItem(ctypes.Structure):
    """Mirror of ``hexkv_work_item`` (32 bytes)."""
    _fields_ = [("row", ctypes.c_int32), ("head_group", ctypes.c_int32), ("part", ctypes.c_int32),
                ("parts", ctypes.c_int32), ("first", ctypes.c_int32), ("count", ctypes.c_int32),
                ("len", ctypes.c_int32), ("heads", ctypes.c_int32)]


class FtAttendParams(ctypes.Structure):
    """Mirror of ``hexkv_ft_attend_params``."""
    _fields_ = [
        ("dtype", ctypes.c_int), ("batch", ctypes.c_int), ("q_heads", ctypes.c_int),
        ("kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int), ("softmax_scale", ctypes.c_float),
        ("q", ctypes.c_void_p), ("q_batch_stride", ctypes.c_int64),
        ("k_new", ctypes.c_void_p), ("v_new", ctypes.c_void_p), ("new_batch_stride", ctypes.c_int64),
        ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p), ("capacity", ctypes.c_int64),
        ("out", ctypes.c_void_p), ("out_batch_stride", ctypes.c_int64),
        ("positions_dev", ctypes.c_void_p), ("position_bias", ctypes.c_int32), ("max_position", ctypes.c_int32),
        ("rotary_dim", ctypes.c_int), ("rotary_base", ctypes.c_float), ("rotary_neox", ctypes.c_int),
        ("partition", ctypes.c_int),
    ]


class Block(ctypes.Structure):
    """Mirror of ``hexkv_block``: depth x height rows of ``width`` bytes."""
    _fields_ = [("data", ctypes.c_void_p), ("width", ctypes.c_int64), ("height", ctypes.c_int64),
                ("depth", ctypes.c_int64), ("row_pitch", ctypes.c_int64), ("slice_pitch", ctypes.c_int64)]


class IpcHandle(ctypes.Structure):
    """Mirror of ``hexkv_ipc_handle``."""
    _fields_ = [("bytes", ctypes.c_ubyte * 64)]


class HexKVError(RuntimeError):
    """A HIP runtime failure reported by the library."""


_lib = None


def load() -> ctypes.CDLL:
    """Load the built library once; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIBRARY.is_file():
        raise RuntimeError(f"{LIBRARY} is missing: build it with `python -m hexgen2_amd.build` "
                           "(the KV data path has no CPU fallback)")
    lib = ctypes.CDLL(str(LIBRARY))
    vp, i64, i32, ci = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int
    ptrs = ctypes.POINTER(ctypes.c_void_p)
    lib.hexkv_version.restype = ci
    lib.hexkv_version.argtypes = []
    lib.hexkv_last_error.restype = ctypes.c_char_p
    lib.hexkv_last_error.argtypes = []
    lib.hexkv_device_status.restype = ci
    lib.hexkv_device_status.argtypes = [ctypes.POINTER(ctypes.c_uint32), ci, vp]
    lib.hexkv_device_xcds.restype = ci
    lib.hexkv_device_xcds.argtypes = [ctypes.POINTER(ctypes.c_int32)]
    for name in ("hexkv_pack", "hexkv_unpack"):
        fn = getattr(lib, name)
        fn.restype = ci
        fn.argtypes = [ptrs, ptrs, ci, ci, i64, i64, i64, ctypes.POINTER(i64), vp]
    lib.hexkv_append.restype = ci
    lib.hexkv_append.argtypes = [vp, vp, ci, i64, i64, i64, vp, i32, vp]
    lib.hexkv_attend_workspace_bytes.restype = ctypes.c_size_t
    lib.hexkv_attend_workspace_bytes.argtypes = [ctypes.POINTER(AttendParams)]
    lib.hexkv_attend_kernel.restype = ctypes.c_int
    lib.hexkv_attend_kernel.argtypes = [ctypes.POINTER(AttendParams)]
    lib.hexkv_attend.restype = ci
    lib.hexkv_attend.argtypes = [ctypes.POINTER(AttendParams), vp, ctypes.c_size_t, vp]
    i32p = ctypes.POINTER(ctypes.c_int32)
    lib.hexkv_attend_plan.restype = ci
    lib.hexkv_attend_plan.argtypes = [ctypes.POINTER(AttendParams), vp, vp, ctypes.c_int32, vp, ctypes.c_int32,
                                      i32p, i32p]
    lib.hexkv_attend_plan_chunk.restype = ci
    lib.hexkv_attend_plan_chunk.argtypes = [ctypes.POINTER(AttendParams), vp, i32p]
    lib.hexkv_attend_plan_kernel.restype = ci
    lib.hexkv_attend_plan_kernel.argtypes = [ctypes.POINTER(AttendParams), vp, i32p]
    lib.hexkv_attend_noalloc.restype = ci
    lib.hexkv_attend_noalloc.argtypes = [ctypes.POINTER(AttendParams), vp]
    blocks = ctypes.POINTER(Block)
    lib.hexkv_flat_concat.restype = ci
    lib.hexkv_flat_concat.argtypes = [blocks, ci, vp, vp]
    lib.hexkv_batch_pad.restype = ci
    lib.hexkv_batch_pad.argtypes = [blocks, ci, ci, ptrs, i64, vp]
    lib.hexkv_head_concat.restype = ci
    lib.hexkv_head_concat.argtypes = [blocks, ci, ci, ptrs, vp]
    u64 = ctypes.c_uint64
    lib.hexkv_ipc_export.restype = ci
    lib.hexkv_ipc_export.argtypes = [vp, ctypes.POINTER(IpcHandle), ctypes.POINTER(u64), ctypes.POINTER(u64)]
    lib.hexkv_ipc_open.restype = ci
    lib.hexkv_ipc_open.argtypes = [ctypes.POINTER(IpcHandle), ctypes.POINTER(vp)]
    lib.hexkv_ipc_close.restype = ci
    lib.hexkv_ipc_close.argtypes = [vp]
    lib.hexkv_ipc_dlpack.restype = vp
    lib.hexkv_ipc_dlpack.argtypes = [vp, u64, ci, ctypes.POINTER(i64), ci, ci, ci]
    lib.hexkv_ft_store.restype = ci
    lib.hexkv_ft_store.argtypes = [vp, i64, i64, i64, vp, vp, ci, ci, i64, ci, ci, ci, vp]
    lib.hexkv_ft_attend_workspace_bytes.restype = ctypes.c_size_t
    lib.hexkv_ft_attend_workspace_bytes.argtypes = [ctypes.POINTER(FtAttendParams)]
    lib.hexkv_ft_attend.restype = ci
    lib.hexkv_ft_attend.argtypes = [ctypes.POINTER(FtAttendParams), vp, ctypes.c_size_t, vp]
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    """Map a hexkv status to the exception type the reference raises for it."""
    if rc == HEXKV_OK:
        return
    message = f"{what}: {load().hexkv_last_error().decode()}"
    if rc in (HEXKV_EINVAL, HEXKV_ERANGE, HEXKV_EWORKSPACE):
        raise ValueError(message)
    if rc == HEXKV_EUNSUPPORTED:
        raise NotImplementedError(message)
    raise HexKVError(message)
