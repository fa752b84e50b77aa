"""Tensor-level entry points of the KV data path, each one call into ``libhexkv.so``.

All tensors live on the current HIP device (``torch.cuda`` on ROCm); work is
enqueued on the current stream.  Shapes follow hexgen_core's cache layout
``[batch, capacity, 2, kv_heads, head_dim]`` (hexgen/hexgen_core/modules/
mha.py:260-265): one *row* is one position's K and V for every KV head.
Lengths that size work (``lens``, ``max_seqlen``) are host integers and are
validated on the host before anything is launched.
"""
from __future__ import annotations

import ctypes
import functools
import math
from collections import OrderedDict
from typing import Optional, Sequence, Union

import torch

from . import _lib

_DTYPES = {torch.float16: _lib.HEXKV_F16, torch.bfloat16: _lib.HEXKV_BF16,
           torch.float32: _lib.HEXKV_F32}

TensorList = Union[torch.Tensor, Sequence[torch.Tensor]]


def _require_device(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if not t.is_cuda:
            raise ValueError("hexkv operates on HIP device tensors only; the KV data path has "
                             f"no CPU fallback (got a tensor on {t.device})")


# torch's own accessor of the current stream's handle (what
# ``torch.cuda.current_stream(device).cuda_stream`` returns, without building
# a Stream object: 0.1 us against 1.9 us a call on MI355X's host).
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t) -> ctypes.c_void_p:
    """The current stream of the device ``t`` (a tensor or ``_Layer``) lives on."""
    if _raw_stream is not None:
        return ctypes.c_void_p(_raw_stream(t.device.index))
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


@functools.lru_cache(maxsize=None)
def device_xcds(index: int) -> int:
    """XCDs (dies with their own L2) of HIP device ``index``
    (``hexkv_device_xcds``): what a work list is planned for when its split
    segments merge inside the attention kernel."""
    n = ctypes.c_int32()
    with torch.cuda.device(index):
        _lib.check(_lib.load().hexkv_device_xcds(ctypes.byref(n)), "hexkv_device_xcds")
    return n.value


_STATUS_TEXT = {
    _lib.STATUS_APPEND_SKIPPED: "an append position read from device memory fell outside the cache, "
                                "so that row was not written",
    _lib.STATUS_LENGTH_CLAMPED: "a sequence length read from device memory exceeded the attended view "
                                "(max_seqlen) and was cut to it, so that row missed keys (with a fused "
                                "append, its own new key)",
    _lib.STATUS_PLACEMENT: "the work items of a split segment ran on more than one XCD, so that segment's "
                           "single-launch merge may have read stale partials",
    _lib.STATUS_LIST: "a work list planned for another attention kernel (another head-group size) was "
                      "launched, and its items were skipped",
}


def device_status(device=None, clear: bool = True) -> int:
    """The HEXKV_STATUS_* flags the kernels raised on ``device`` (default:
    the current one) since the last clear, after the current stream's work
    has finished; resets them when ``clear``."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    flags = ctypes.c_uint32()
    with torch.cuda.device(dev):
        rc = _lib.load().hexkv_device_status(ctypes.byref(flags), 1 if clear else 0,
                                             ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
    _lib.check(rc, "hexkv_device_status")
    return flags.value


def check_device_status(device=None) -> None:
    """Raise ValueError if a kernel met out-of-contract values in device
    memory since the last check (clearing the flags): the device-side
    counterpart of the reference's capacity assert (hexgen/hexgen_core/
    modules/mha.py:281-282).  It synchronises, so callers run it where they
    synchronise anyway (after reading a token)."""
    flags = device_status(device, clear=True) & _lib.STATUS_ERRORS
    if flags:
        text = "; ".join(t for bit, t in _STATUS_TEXT.items() if flags & bit)
        raise ValueError(f"hexkv device status {flags:#x}: {text}")


def _contiguous(shape, stride) -> bool:
    """``Tensor.is_contiguous()`` of a view with these sizes and strides,
    without building the view (size-1 dims are free; an empty view is
    contiguous)."""
    if 0 in shape:
        return True
    expected = 1
    for n, st in zip(reversed(shape), reversed(stride)):
        if n != 1 and st != expected:
            return False
        expected *= n
    return True


@functools.lru_cache(maxsize=256)
def _row_geometry_of(shape, stride, elem_size: int):
    """(row_elems, row_bytes, seq_stride_rows) of a ``[B, S, *row]`` cache
    given as sizes and strides."""
    if len(shape) < 3:
        raise ValueError(f"cache must be [batch, capacity, *row], got shape {tuple(shape)}")
    row_elems = math.prod(shape[2:])
    if shape[0] and shape[1] and not _contiguous(shape[2:], stride[2:]):
        raise ValueError("cache rows (dims 2+) must be contiguous")
    if shape[1] > 1 and stride[1] != row_elems:
        raise ValueError("cache positions must be consecutive rows (stride(1) == row size)")
    if shape[0] > 1 and stride[0] % row_elems:
        raise ValueError("cache batch stride must be a whole number of rows")
    seq_stride = stride[0] // row_elems if shape[0] > 1 else shape[1]
    return row_elems, row_elems * elem_size, seq_stride


def _row_geometry(cache: torch.Tensor):
    """(row_elems, row_bytes, seq_stride_rows) of a ``[B, S, *row]`` cache."""
    return _row_geometry_of(tuple(cache.shape), cache.stride(), cache.element_size())


class _Layer:
    """Shape, dtype and device of one cache layer (``[B, S, *row]``)."""

    __slots__ = ("shape", "dtype", "device")

    def __init__(self, shape, dtype, device):
        self.shape, self.dtype, self.device = shape, dtype, device


def _as_layers(x: TensorList) -> list:
    return list(x.unbind(0)) if isinstance(x, torch.Tensor) else list(x)


def _check_lens(lens: Sequence[int], batch: int) -> list:
    lens = [int(n) for n in lens]
    if len(lens) != batch:
        raise ValueError(f"{len(lens)} lengths for a batch of {batch}")
    return lens


_LAYER_ARRAYS: "OrderedDict[tuple, ctypes.Array]" = OrderedDict()


def _layer_ptrs(stacked: torch.Tensor) -> ctypes.Array:
    """Base address of each layer of a stacked ``[n_layers, ...]`` tensor, as
    the ``void *[]`` the C entry points take.  The array depends only on
    (address, layer stride, layer count), so recently used ones are kept and
    handed out again (the C side only reads them)."""
    key = (stacked.data_ptr(), stacked.stride(0) * stacked.element_size(), stacked.shape[0])
    arr = _LAYER_ARRAYS.get(key)
    if arr is None:
        base, step, n = key
        arr = (ctypes.c_void_p * n)(*[base + l * step for l in range(n)])
        _LAYER_ARRAYS[key] = arr
        if len(_LAYER_ARRAYS) > 64:
            _LAYER_ARRAYS.popitem(last=False)
    return arr


def _ptr_array(ptrs: list) -> ctypes.Array:
    return (ctypes.c_void_p * len(ptrs))(*ptrs)


def _packed_ptrs(packed: TensorList, n_layers: int, total: int, row_elems: int, dtype, device):
    if isinstance(packed, torch.Tensor):
        # Stacked [n_layers, total, *row]: checked once, addressed per layer.
        _require_device(packed)
        if packed.dtype != dtype or packed.device != device:
            raise ValueError("packed and cache tensors differ in dtype or device")
        if packed.dim() < 1 or packed.shape[0] != n_layers:
            raise ValueError(f"packed tensor of shape {tuple(packed.shape)} for {n_layers} cache layers")
        shape, stride = tuple(packed.shape[1:]), packed.stride()[1:]
        if math.prod(shape) != total * row_elems or not _contiguous(shape, stride):
            raise ValueError(f"packed layer must be contiguous with {total} rows of {row_elems} "
                             f"elements, got shape {shape}")
        return _layer_ptrs(packed)
    layers = list(packed)
    if len(layers) != n_layers:
        raise ValueError(f"{len(layers)} packed layers for {n_layers} cache layers")
    ptrs = []
    for t in layers:
        _require_device(t)
        if t.dtype != dtype or t.device != device:
            raise ValueError("packed and cache tensors differ in dtype or device")
        if t.numel() != total * row_elems or not t.is_contiguous():
            raise ValueError(f"packed layer must be contiguous with {total} rows of {row_elems} "
                             f"elements, got shape {tuple(t.shape)}")
        ptrs.append(t.data_ptr())
    return _ptr_array(ptrs)


def _cache_ptrs(cache_layers: TensorList):
    """(first layer's shape/dtype/device, per-layer base addresses, row
    geometry) of the cache layers: a list of ``[B, S, *row]`` tensors sharing
    shape, strides, dtype and device, or one stacked ``[n_layers, B, S,
    *row]`` tensor (checked from its sizes and strides, no views built)."""
    if isinstance(cache_layers, torch.Tensor):
        if cache_layers.dim() < 1 or cache_layers.shape[0] == 0:
            raise ValueError("no cache layers")
        _require_device(cache_layers)
        shape = tuple(cache_layers.shape[1:])
        geometry = _row_geometry_of(shape, cache_layers.stride()[1:], cache_layers.element_size())
        return _Layer(shape, cache_layers.dtype, cache_layers.device), _layer_ptrs(cache_layers), geometry
    layers = list(cache_layers)
    if not layers:
        raise ValueError("no cache layers")
    first = layers[0]
    _require_device(first)
    geometry = _row_geometry(first)
    for t in layers[1:]:
        _require_device(t)
        if t.shape != first.shape or t.dtype != first.dtype or t.device != first.device \
                or t.stride() != first.stride():
            raise ValueError("all cache layers must share shape, strides, dtype and device")
    return _Layer(tuple(first.shape), first.dtype, first.device), _ptr_array([t.data_ptr() for t in layers]), geometry


def pack_live(cache_layers: TensorList, lens: Sequence[int],
              out: Optional[TensorList] = None) -> TensorList:
    """Gather rows ``[0, lens[b])`` of every sequence of every layer into the
    packed handoff layout ``[n_layers, sum(lens), *row]`` (one launch).

    Batch-1 form of hexgen2/model.py:81 ``t[:, :L].contiguous()`` per layer,
    generalised to ragged batches.  ``cache_layers`` is a list of per-layer
    ``[B, S, *row]`` caches or one stacked ``[n_layers, B, S, *row]`` tensor
    (checked once, the cheaper form for many layers); ``out`` may be one
    ``[n_layers, T, *row]`` tensor or a list of per-layer contiguous tensors.
    """
    first, layers, (row_elems, row_bytes, seq_stride) = _cache_ptrs(cache_layers)
    lens = _check_lens(lens, first.shape[0])
    total = sum(lens)
    if out is None:
        out = torch.empty((len(layers), total, *first.shape[2:]), dtype=first.dtype,
                          device=first.device)
    dst = _packed_ptrs(out, len(layers), total, row_elems, first.dtype, first.device)
    rc = _lib.load().hexkv_pack(layers, dst, len(layers), len(lens), seq_stride,
                                first.shape[1], row_bytes, (ctypes.c_int64 * len(lens))(*lens),
                                _stream(first))
    _lib.check(rc, "hexkv_pack")
    return out


def unpack_live(packed: TensorList, cache_layers: TensorList, lens: Sequence[int]) -> None:
    """Scatter the packed handoff layout into preallocated caches: rows
    ``[0, lens[b])`` of each sequence are overwritten, all other rows are
    left untouched (hexgen2/model.py:104-108 writes into ``torch.empty``)."""
    first, layers, (row_elems, row_bytes, seq_stride) = _cache_ptrs(cache_layers)
    lens = _check_lens(lens, first.shape[0])
    src = _packed_ptrs(packed, len(layers), sum(lens), row_elems, first.dtype, first.device)
    rc = _lib.load().hexkv_unpack(src, layers, len(layers),
                                  len(lens), seq_stride, first.shape[1], row_bytes,
                                  (ctypes.c_int64 * len(lens))(*lens), _stream(first))
    _lib.check(rc, "hexkv_unpack")


def append_kv(cache: torch.Tensor, kv_new: torch.Tensor, positions: Optional[torch.Tensor] = None,
              position_bias: int = 0) -> None:
    """Write ``kv_new[b]`` (one row per sequence) into ``cache[b, pos_b]`` with
    ``pos_b = positions[b] + position_bias`` (``positions`` a device int32
    tensor, or None for a batch-uniform position): hexgen/hexgen_core/modules/
    mha.py:286 with per-sequence offsets."""
    _require_device(cache, kv_new)
    row_elems, row_bytes, seq_stride = _row_geometry(cache)
    batch = kv_new.shape[0]
    if kv_new.dtype != cache.dtype or kv_new.device != cache.device:
        raise ValueError("kv_new and cache differ in dtype or device")
    if kv_new.numel() != batch * row_elems or not kv_new.is_contiguous():
        raise ValueError(f"kv_new must be contiguous [batch, *row], got {tuple(kv_new.shape)}")
    if batch > cache.shape[0]:
        raise ValueError(f"batch {batch} exceeds the cache's {cache.shape[0]} sequences")
    pos_ptr = None
    if positions is not None:
        _require_device(positions)
        if positions.dtype != torch.int32 or positions.numel() < batch or not positions.is_contiguous():
            raise ValueError("positions must be a contiguous int32 device tensor with one entry per sequence")
        pos_ptr = positions.data_ptr()
    rc = _lib.load().hexkv_append(kv_new.data_ptr(), cache.data_ptr(), batch, seq_stride,
                                  cache.shape[1], row_bytes, pos_ptr, int(position_bias),
                                  _stream(cache))
    _lib.check(rc, "hexkv_append")


def _attend_params(q, cache, out, seqlens, seqlen_bias, max_seqlen, kv_new, causal,
                   softmax_scale, partition, kernel="auto") -> _lib.AttendParams:
    if q.dim() != 4 or cache.dim() != 5 or cache.shape[2] != 2:
        raise ValueError("q must be [batch, q_len, q_heads, head_dim] and the cache "
                         "[batch, capacity, 2, kv_heads, head_dim]")
    batch, q_len, q_heads, head_dim = q.shape
    if q.dtype not in _DTYPES or cache.dtype != q.dtype or out.dtype != q.dtype:
        raise ValueError("q, cache and out must share one of float16, bfloat16, float32")
    if cache.shape[0] < batch or cache.shape[4] != head_dim:
        raise ValueError(f"cache shape {tuple(cache.shape)} does not fit q {tuple(q.shape)}")
    kv_heads = cache.shape[3]
    if q_heads % kv_heads:
        raise ValueError("q_heads must be a multiple of kv_heads")
    if out.shape != q.shape:
        raise ValueError(f"out shape {tuple(out.shape)} differs from q shape {tuple(q.shape)}")
    qs, os_, cs = q.stride(), out.stride(), cache.stride()
    if qs[3] != 1 or qs[2] != head_dim:
        raise ValueError("q heads must be contiguous [.., heads, head_dim]")
    if os_[3] != 1 or os_[2] != head_dim:
        raise ValueError("out heads must be contiguous [.., heads, head_dim]")
    if cs[4] != 1 or cs[3] != head_dim:
        raise ValueError("cache heads must be contiguous [.., kv_heads, head_dim]")
    p = _lib.AttendParams()
    p.dtype = _DTYPES[q.dtype]
    p.batch, p.q_len, p.q_heads, p.kv_heads, p.head_dim = batch, q_len, q_heads, kv_heads, head_dim
    p.causal = 1 if causal else 0
    p.softmax_scale = float(head_dim ** -0.5 if softmax_scale is None else softmax_scale)
    p.q, p.q_batch_stride, p.q_row_stride = q.data_ptr(), qs[0], qs[1]
    p.cache = cache.data_ptr()
    p.cache_batch_stride, p.cache_pos_stride, p.cache_kv_stride = cs[0], cs[1], cs[2]
    p.capacity = cache.shape[1]
    p.out, p.out_batch_stride, p.out_row_stride = out.data_ptr(), os_[0], os_[1]
    if seqlens is not None:
        _require_device(seqlens)
        if seqlens.dtype != torch.int32 or seqlens.numel() < batch or not seqlens.is_contiguous():
            raise ValueError("seqlens must be a contiguous int32 device tensor")
        p.seqlens_dev = seqlens.data_ptr()
    p.seqlen_bias = int(seqlen_bias)
    p.max_seqlen = int(max_seqlen)
    if kv_new is not None:
        _require_device(kv_new)
        if kv_new.dtype != q.dtype or kv_new.numel() != batch * 2 * kv_heads * head_dim \
                or not kv_new.is_contiguous():
            raise ValueError("kv_new must be contiguous [batch, 2, kv_heads, head_dim]")
        p.kv_new = kv_new.data_ptr()
    p.partition = int(partition)
    if kernel not in _lib.KERNELS:
        raise ValueError(f"kernel must be one of {sorted(_lib.KERNELS)}, got {kernel!r}")
    p.kernel = _lib.KERNELS[kernel]
    return p


def attend_workspace_bytes(q: torch.Tensor, cache: torch.Tensor, max_seqlen: int,
                           partition: int = 0, kernel: str = "auto") -> int:
    out = q  # geometry only
    p = _attend_params(q, cache, out, None, max_seqlen, max_seqlen, None, False, None, partition, kernel)
    return int(_lib.load().hexkv_attend_workspace_bytes(ctypes.byref(p)))


def attend_kernel(q: torch.Tensor, cache: torch.Tensor, kernel: str = "auto") -> str:
    """Name of the kernel ("valu" or "mfma") ``decode_attention`` runs for
    this geometry and ``kernel`` choice."""
    p = _attend_params(q, cache, q, None, 1, 1, None, False, None, 0, kernel)
    rc = int(_lib.load().hexkv_attend_kernel(ctypes.byref(p)))
    _lib.check(min(rc, 0), "hexkv_attend_kernel")
    return {v: k for k, v in _lib.KERNELS.items()}[rc]


def decode_attention(q: torch.Tensor, cache: torch.Tensor, *, max_seqlen: int,
                     seqlens: Optional[torch.Tensor] = None, seqlen_bias: int = 0,
                     kv_new: Optional[torch.Tensor] = None, causal: bool = False,
                     softmax_scale: Optional[float] = None, out: Optional[torch.Tensor] = None,
                     workspace: Optional[torch.Tensor] = None, partition: int = 0,
                     kernel: str = "auto", lens: Optional[Sequence[int]] = None,
                     single_launch: bool = True) -> torch.Tensor:
    """Attention of ``q [B, q_len, Hq, D]`` over a cache ``[B, S, 2, Hkv, D]``.

    Sequence b attends to ``len_b = seqlens[b] + seqlen_bias`` keys (the
    uniform ``seqlen_bias`` alone when ``seqlens`` is None); with ``kv_new``
    ``[B, 2, Hkv, D]`` the row is first appended at position ``len_b`` and
    ``len_b + 1`` keys are attended.  ``max_seqlen`` is a host bound on the
    attended length (including that +1).  GQA maps q head h to KV head
    ``h // (Hq // Hkv)`` (mha.py:223-224); ``softmax_scale`` defaults to
    ``D ** -0.5`` (gpt.py:72).  ``kernel`` picks the score kernel: "valu"
    (packed dot products), "mfma" (the GQA group on the matrix cores, 16-bit
    only) or "auto" (the library's choice).  ``lens``, the host values of
    ``seqlens`` (decode rows), makes the call run a work list
    (``hexkv_attend_plan``; ``partition`` then sets its chunk size).  With
    ``single_launch`` the list is planned for the device's XCDs and split rows
    merge inside the attention kernel (one launch); otherwise a second kernel
    merges them.  A caller-supplied ``workspace`` must have been zeroed once
    after allocation (its leading counter words; every call leaves them zero).
    """
    _require_device(q, cache)
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    p = _attend_params(q, cache, out, seqlens, seqlen_bias, max_seqlen, kv_new, causal,
                       softmax_scale, partition, kernel)
    lib = _lib.load()
    work = None
    if lens is not None:
        work = _plan_work(p, lens, q.device, single_launch)  # kept alive until the launch is enqueued
        work.apply(p)
    need = int(lib.hexkv_attend_workspace_bytes(ctypes.byref(p)))
    ws_ptr, ws_bytes = None, 0
    if need:
        if workspace is None or workspace.numel() * workspace.element_size() < need:
            workspace = torch.zeros(need, dtype=torch.uint8, device=q.device)
        _require_device(workspace)
        ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    rc = lib.hexkv_attend(ctypes.byref(p), ws_ptr, ws_bytes, _stream(q))
    _lib.check(rc, "hexkv_attend")
    return out


class WorkList:
    """A ``hexkv_attend_plan`` work list in device memory: ``items``
    (``[n_items, 8]`` int32, one ``hexkv_work_item`` per workgroup) and
    ``parts`` (partitions per (row, head group)), valid for the lengths and
    ``seqlen_bias``/``max_seqlen`` it was built for.  ``kernel`` is the
    ``hexkv_attend_params.kernel`` value it was planned with (the row-block
    kernel plans other head groups), which launches of the list use."""

    def __init__(self, items: torch.Tensor, parts: torch.Tensor, n_items: int, max_parts: int, xcds: int = 0,
                 kernel: int = 0):
        self.items, self.parts, self.n_items, self.max_parts = items, parts, n_items, max_parts
        self.xcds, self.kernel = xcds, kernel

    def apply(self, p: _lib.AttendParams) -> None:
        p.work_items_dev, p.work_parts_dev = self.items.data_ptr(), self.parts.data_ptr()
        p.n_work_items, p.work_max_parts, p.work_xcds = self.n_items, self.max_parts, self.xcds
        p.kernel = self.kernel


def _kernel_group(group: int) -> int:
    """Query heads per workgroup for a GQA group (the library's rule)."""
    for g in (8, 4, 2, 1):
        if group % g == 0:
            return g
    return 1


def _plan_xcds(p: _lib.AttendParams, device, single_launch: bool) -> int:
    """work_xcds for a list of these parameters: the device's XCD count when
    split segments are to merge in the attention kernel (and the counters
    cover every segment), else 0."""
    if not single_launch:
        return 0
    groups = p.q_heads // _kernel_group(p.q_heads // p.kv_heads)
    if p.batch * groups > _lib.ATTEND_COUNTER_WORDS:
        return 0
    xcds = device_xcds(torch.device(device).index or 0)
    return xcds if 1 < xcds <= 8 else 0


def _plan_kernel(p: _lib.AttendParams, c_lens) -> int:
    """The kernel value to plan and launch a list over these lengths with
    (``hexkv_attend_plan_kernel``: the requested one, or for "auto" the
    row-block kernel on large calls planned for the XCDs)."""
    kernel = ctypes.c_int32()
    _lib.check(_lib.load().hexkv_attend_plan_kernel(ctypes.byref(p), c_lens, ctypes.byref(kernel)),
               "hexkv_attend_plan_kernel")
    return kernel.value


def _plan_work(p: _lib.AttendParams, lens: Sequence[int], device, single_launch: bool = True) -> WorkList:
    """Build the work list on the host (``hexkv_attend_plan``) and copy it to
    ``device`` on the current stream (asynchronously, from pinned memory).
    Refused under graph capture: the capture would record a copy from a
    temporary host buffer, replayed later with whatever it then holds (a
    captured decode step takes its lists from ``StepWorkLists``)."""
    if torch.cuda.is_current_stream_capturing():
        raise ValueError("work lists cannot be planned under graph capture: build them before capture "
                         "(StepWorkLists, AttendPlan.fix_work_list, DecodeStepGraph(lens=...))")
    lib = _lib.load()
    if len(lens) != p.batch:
        raise ValueError(f"{len(lens)} host lengths for a batch of {p.batch}")
    p.work_xcds = _plan_xcds(p, device, single_launch)
    c_lens = (ctypes.c_int32 * len(lens))(*[int(n) for n in lens])
    requested = p.kernel
    p.kernel = _plan_kernel(p, c_lens)
    try:
        n_items, max_parts = ctypes.c_int32(), ctypes.c_int32()
        _lib.check(lib.hexkv_attend_plan(ctypes.byref(p), c_lens, None, 0, None, 0, ctypes.byref(n_items),
                                         ctypes.byref(max_parts)), "hexkv_attend_plan")
        n_segs = p.batch * p.q_heads  # head groups never outnumber query heads
        items = torch.empty((max(n_items.value, 1), 8), dtype=torch.int32, pin_memory=True)
        parts = torch.empty(max(n_segs, 1), dtype=torch.int32, pin_memory=True)
        _lib.check(lib.hexkv_attend_plan(ctypes.byref(p), c_lens, ctypes.c_void_p(items.data_ptr()),
                                         items.shape[0], ctypes.c_void_p(parts.data_ptr()), parts.shape[0],
                                         ctypes.byref(n_items), ctypes.byref(max_parts)), "hexkv_attend_plan")
        return WorkList(items.to(device, non_blocking=True), parts.to(device, non_blocking=True),
                        n_items.value, max_parts.value, p.work_xcds, p.kernel)
    finally:
        p.kernel = requested


def decode_attention_noalloc(q: torch.Tensor, cache: torch.Tensor, out: torch.Tensor, *, max_seqlen: int,
                             seqlens: Optional[torch.Tensor] = None, seqlen_bias: int = 0,
                             kv_new: Optional[torch.Tensor] = None, causal: bool = False,
                             softmax_scale: Optional[float] = None, partition: int = 0,
                             kernel: str = "auto") -> torch.Tensor:
    """``decode_attention`` through ``hexkv_attend_noalloc``: no workspace and
    no allocation (the split-K partials go to the library's static per-GPU
    scratch of ``_lib.NOALLOC_SCRATCH_BYTES``); ``out`` is required.  Calls
    on one GPU share that scratch, so overlapping calls on different streams
    race.  Raises ValueError when the call needs more scratch than there is."""
    _require_device(q, cache, out)
    p = _attend_params(q, cache, out, seqlens, seqlen_bias, max_seqlen, kv_new, causal,
                       softmax_scale, partition, kernel)
    _lib.check(_lib.load().hexkv_attend_noalloc(ctypes.byref(p), _stream(q)), "hexkv_attend_noalloc")
    return out


def ft_pack(dtype: torch.dtype) -> int:
    """Elements per 16-byte K chunk of the FT layout: 4 for float32, 8 for
    16-bit data (mha.py:423, generation.py:317)."""
    return 4 if dtype == torch.float32 else 8


def ft_cache_shapes(batch: int, kv_heads: int, capacity: int, head_dim: int, dtype: torch.dtype):
    """(K shape, V shape) of one layer's FT cache:
    ``[batch, kv_heads, head_dim // pack, capacity, pack]`` and
    ``[batch, kv_heads, capacity, head_dim]`` (mha.py:420-427)."""
    pack = ft_pack(dtype)
    if head_dim % pack:
        raise ValueError(f"head_dim {head_dim} is not a multiple of the FT pack size {pack}")
    return (batch, kv_heads, head_dim // pack, capacity, pack), (batch, kv_heads, capacity, head_dim)


def _check_ft_caches(k_cache: torch.Tensor, v_cache: torch.Tensor):
    """(batch, kv_heads, capacity, head_dim) of a contiguous FT cache pair."""
    if k_cache.dim() != 5 or v_cache.dim() != 4:
        raise ValueError("FT caches are K [B, Hkv, D/pack, S, pack] and V [B, Hkv, S, D]")
    batch, kv_heads, capacity, head_dim = v_cache.shape
    if tuple(k_cache.shape) != ft_cache_shapes(batch, kv_heads, capacity, head_dim, v_cache.dtype)[0]:
        raise ValueError(f"FT K cache {tuple(k_cache.shape)} does not match V cache {tuple(v_cache.shape)}")
    if k_cache.dtype != v_cache.dtype or v_cache.dtype not in _DTYPES:
        raise ValueError("FT caches must share one of float16, bfloat16, float32")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("FT caches must be contiguous (batch slices of them are)")
    return batch, kv_heads, capacity, head_dim


def ft_store(kv: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor) -> None:
    """Write ``kv [B, s, 2, Hkv, D]`` into positions ``[0, s)`` of the FT
    caches (one launch, a bit copy): the FT branch of _update_kv_cache,
    mha.py:289-305."""
    _require_device(kv, k_cache, v_cache)
    batch, kv_heads, capacity, head_dim = _check_ft_caches(k_cache, v_cache)
    if kv.dim() != 5 or kv.shape[2] != 2 or kv.shape[3] != kv_heads or kv.shape[4] != head_dim \
            or kv.shape[0] != batch:
        raise ValueError(f"kv {tuple(kv.shape)} does not fit FT caches of {batch} x {kv_heads} x {head_dim}")
    if kv.dtype != v_cache.dtype or kv.device != v_cache.device:
        raise ValueError("kv and the caches differ in dtype or device")
    if kv.stride(4) != 1 or kv.stride(3) != head_dim:
        kv = kv.contiguous()
    rc = _lib.load().hexkv_ft_store(kv.data_ptr(), kv.stride(0), kv.stride(1), kv.stride(2),
                                    k_cache.data_ptr(), v_cache.data_ptr(), batch, kv.shape[1], capacity,
                                    kv_heads, head_dim, _DTYPES[kv.dtype], _stream(kv))
    _lib.check(rc, "hexkv_ft_store")


def _ft_params(q, k_new, v_new, k_cache, v_cache, out, positions, position_bias, max_position,
               rotary_dim, rotary_base, rotary_neox, softmax_scale, partition) -> _lib.FtAttendParams:
    batch, kv_heads, capacity, head_dim = _check_ft_caches(k_cache, v_cache)
    if q.dim() != 3 or q.shape[0] != batch or q.shape[2] != head_dim or q.shape[1] % kv_heads:
        raise ValueError(f"q {tuple(q.shape)} must be [batch, q_heads, head_dim] over FT caches of "
                         f"{batch} x {kv_heads} x {head_dim}")
    for name, t in (("k_new", k_new), ("v_new", v_new)):
        if tuple(t.shape) != (batch, kv_heads, head_dim):
            raise ValueError(f"{name} {tuple(t.shape)} must be [batch, kv_heads, head_dim]")
    if k_new.stride() != v_new.stride():
        raise ValueError("k_new and v_new must share strides")
    if out.shape != q.shape:
        raise ValueError(f"out shape {tuple(out.shape)} differs from q shape {tuple(q.shape)}")
    for name, t in (("q", q), ("k_new", k_new), ("out", out)):
        if t.dtype != v_cache.dtype:
            raise ValueError(f"{name} dtype differs from the caches")
        if t.stride(2) != 1 or t.stride(1) != head_dim:
            raise ValueError(f"{name} heads must be contiguous [.., heads, head_dim]")
    p = _lib.FtAttendParams()
    p.dtype = _DTYPES[q.dtype]
    p.batch, p.q_heads, p.kv_heads, p.head_dim = batch, q.shape[1], kv_heads, head_dim
    p.softmax_scale = float(head_dim ** -0.5 if softmax_scale is None else softmax_scale)
    p.q, p.q_batch_stride = q.data_ptr(), q.stride(0)
    p.k_new, p.v_new, p.new_batch_stride = k_new.data_ptr(), v_new.data_ptr(), k_new.stride(0)
    p.k_cache, p.v_cache, p.capacity = k_cache.data_ptr(), v_cache.data_ptr(), capacity
    p.out, p.out_batch_stride = out.data_ptr(), out.stride(0)
    if positions is not None:
        _require_device(positions)
        if positions.dtype != torch.int32 or positions.numel() < batch or not positions.is_contiguous():
            raise ValueError("positions must be a contiguous int32 device tensor")
        p.positions_dev = positions.data_ptr()
    p.position_bias = int(position_bias)
    p.max_position = int(max_position)
    p.rotary_dim, p.rotary_base, p.rotary_neox = int(rotary_dim), float(rotary_base), 1 if rotary_neox else 0
    p.partition = int(partition)
    return p


def ft_attend_workspace_bytes(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                              max_position: int, partition: int = 0) -> int:
    """Workspace bytes ``ft_attend`` needs for this geometry and bound."""
    batch, kv_heads, _, head_dim = _check_ft_caches(k_cache, v_cache)
    new = q.new_empty((batch, kv_heads, head_dim))
    p = _ft_params(q, new, new, k_cache, v_cache, q, None, 0, max_position, 0, 10000.0, True, None, partition)
    return int(_lib.load().hexkv_ft_attend_workspace_bytes(ctypes.byref(p)))


def ft_attend(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, k_cache: torch.Tensor,
              v_cache: torch.Tensor, *, max_position: int, positions: Optional[torch.Tensor] = None,
              position_bias: int = 0, rotary_dim: int = 0, rotary_base: float = 10000.0,
              rotary_neox: bool = True, softmax_scale: Optional[float] = None,
              out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None,
              partition: int = 0) -> torch.Tensor:
    """One decode step over FT caches (one launch plus the split merge):
    rotate ``q [B, Hq, D]`` and ``k_new [B, Hkv, D]`` at position
    ``pos_b = positions[b] + position_bias`` (``position_bias`` alone when
    ``positions`` is None), write ``k_new``/``v_new`` at ``pos_b``, attend over
    ``[0, pos_b]``.  The semantics of ft_attention.single_query_attention as
    mha.py:310-337 calls it; ``max_position`` is a host bound on every
    ``pos_b`` (below the cache capacity)."""
    _require_device(q, k_new, v_new, k_cache, v_cache)
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    p = _ft_params(q, k_new, v_new, k_cache, v_cache, out, positions, position_bias, max_position,
                   rotary_dim, rotary_base, rotary_neox, softmax_scale, partition)
    lib = _lib.load()
    need = int(lib.hexkv_ft_attend_workspace_bytes(ctypes.byref(p)))
    ws_ptr, ws_bytes = None, 0
    if need:
        if workspace is None or workspace.numel() * workspace.element_size() < need:
            workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
        _require_device(workspace)
        ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    rc = lib.hexkv_ft_attend(ctypes.byref(p), ws_ptr, ws_bytes, _stream(q))
    _lib.check(rc, "hexkv_ft_attend")
    return out


def _tensor_geometry(t: Optional[torch.Tensor]):
    """Everything about a tensor a prebuilt parameter block depends on apart
    from its address: shape, strides (which fix its contiguity), dtype and
    device.  A GPU tensor's device is its index (``get_device``, cheap: this
    key is built on every ``AttendPlan`` call), any other tensor's its
    device type."""
    if t is None:
        return None
    dev = t.get_device()
    return t.shape, t.stride(), t.dtype, dev if dev >= 0 else t.device.type


def _plan_geometry(q, cache, out, kv_new) -> tuple:
    """The key an ``AttendPlan`` compares per call: the geometry of q, cache,
    out and kv_new (None when the call has no fused append)."""
    return _tensor_geometry(q), _tensor_geometry(cache), _tensor_geometry(out), _tensor_geometry(kv_new)


def _check_plan_geometry(want: tuple, got: tuple) -> None:
    """Raise ValueError naming the first tensor whose geometry differs from
    the plan's."""
    if want == got:
        return
    for name, a, b in zip(("q", "cache", "out", "kv_new"), want, got):
        if a != b:
            if a is None or b is None:
                raise ValueError("AttendPlan built with kv_new must be called with kv_new, and only then")
            raise ValueError(f"AttendPlan called with a different {name} geometry: "
                             f"built for shape/strides/dtype/device/contiguous {a}, got {b}")


class AttendPlan:
    """Prebuilt ``hexkv_attend`` parameters for a decode loop on one geometry.

    Building the parameter block once and patching only pointers, the length
    bias and ``max_seqlen`` per call keeps host overhead per layer small; the
    workspace is allocated (zeroed) once for the largest ``max_seqlen`` the
    loop will use.  Every call checks that q, cache, out and kv_new have
    exactly the geometry (shape, strides, dtype, device) the block was built
    for, since only their addresses are patched.  Each call launches on the
    current stream, so a call inside graph capture is recorded into the graph
    -- with a work list fixed beforehand (``fix_work_list``): planning one
    under capture is refused.  Arguments as for ``decode_attention``; a plan
    built with ``kv_new`` is called with one.
    """

    def __init__(self, q: torch.Tensor, cache: torch.Tensor, out: torch.Tensor, *,
                 max_seqlens: Sequence[int], seqlens: Optional[torch.Tensor] = None,
                 kv_new: Optional[torch.Tensor] = None, softmax_scale: Optional[float] = None,
                 partition: int = 0, kernel: str = "auto", lens: Optional[Sequence[int]] = None,
                 single_launch: bool = True):
        """``lens``: the host values of ``seqlens`` (decode rows).  With them
        each call runs a work list (``hexkv_attend_plan``: compact, largest
        items first) built once per (``seqlen_bias``, ``max_seqlen``) and
        shared by every layer called with the same pair; without them the
        library's uniform partitions over the device lengths."""
        _require_device(q, cache, out)
        self.params = _attend_params(q, cache, out, seqlens, 0, max(max_seqlens), kv_new, False,
                                     softmax_scale, partition, kernel)
        self.lib = _lib.load()
        need = 0
        if lens is None:
            for m in max_seqlens:
                self.params.max_seqlen = int(m)
                need = max(need, int(self.lib.hexkv_attend_workspace_bytes(ctypes.byref(self.params))))
        self.workspace = torch.zeros(max(need, 16), dtype=torch.uint8, device=q.device)
        self.ws_ptr, self.ws_bytes = self.workspace.data_ptr(), self.workspace.numel()
        self.device = q.device
        self.fused = kv_new is not None
        self.single_launch = single_launch
        self.geometry = _plan_geometry(q, cache, out, kv_new)
        self.lens = None if lens is None else [int(n) for n in lens]
        self.work_key, self.work = None, None
        self.kernel = self.params.kernel  # as requested; a work list sets the one its launches use

    def _grow_workspace(self) -> None:
        need = int(self.lib.hexkv_attend_workspace_bytes(ctypes.byref(self.params)))
        if need > self.ws_bytes:
            self.workspace = torch.zeros(need, dtype=torch.uint8, device=self.device)
            self.ws_ptr, self.ws_bytes = self.workspace.data_ptr(), need

    def _use_work_list(self, seqlen_bias: int, max_seqlen: int) -> None:
        """Point the parameter block at the work list for this step (built
        on first use) and grow the workspace if the list needs more."""
        p = self.params
        key = (int(seqlen_bias), int(max_seqlen))
        if key != self.work_key:
            p.work_items_dev, p.kernel = None, self.kernel
            self.work = _plan_work(p, self.lens, self.device, self.single_launch)
            self.work_key = key
        self.work.apply(p)
        self._grow_workspace()

    def fix_work_list(self, work: WorkList) -> None:
        """Run every later call on ``work`` (until the next ``fix_work_list``):
        the per-call list building stops, and the workspace grows to fit the
        list.  A workspace a captured graph holds must already fit: size it
        first with ``reserve``."""
        p = self.params
        self.lens, self.work_key, self.work = None, None, work
        work.apply(p)
        self._grow_workspace()

    def reserve(self, lists: Sequence[WorkList]) -> None:
        """Grow the workspace once to fit every list in ``lists``."""
        p = self.params
        saved = (p.work_items_dev, p.work_parts_dev, p.n_work_items, p.work_max_parts, p.work_xcds, p.kernel)
        for work in lists:
            work.apply(p)
            self._grow_workspace()
        (p.work_items_dev, p.work_parts_dev, p.n_work_items, p.work_max_parts, p.work_xcds, p.kernel) = saved

    def check(self, q: torch.Tensor, cache: torch.Tensor, out: torch.Tensor,
              kv_new: Optional[torch.Tensor]) -> None:
        """Raise ValueError unless the tensors match the plan's geometry."""
        _check_plan_geometry(self.geometry, _plan_geometry(q, cache, out, kv_new))

    def __call__(self, q: torch.Tensor, cache: torch.Tensor, out: torch.Tensor,
                 kv_new: Optional[torch.Tensor], seqlen_bias: int, max_seqlen: int,
                 lengths_out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """One call; ``lengths_out`` (work lists with kv_new: a contiguous int32
        device tensor with one entry per row) receives each row's new length."""
        self.check(q, cache, out, kv_new)
        p = self.params
        p.q, p.cache, p.out = q.data_ptr(), cache.data_ptr(), out.data_ptr()
        if kv_new is not None:
            p.kv_new = kv_new.data_ptr()
        p.seqlen_bias, p.max_seqlen = int(seqlen_bias), int(max_seqlen)
        if self.lens is not None:
            self._use_work_list(seqlen_bias, max_seqlen)
        if lengths_out is not None:
            _require_device(lengths_out)
            if lengths_out.dtype != torch.int32 or lengths_out.numel() < p.batch or not lengths_out.is_contiguous():
                raise ValueError("lengths_out must be a contiguous int32 device tensor with one entry per row")
            p.lengths_out_dev = lengths_out.data_ptr()
        try:
            rc = self.lib.hexkv_attend(ctypes.byref(p), self.ws_ptr, self.ws_bytes, _stream(q))
        finally:
            p.lengths_out_dev = None
        _lib.check(rc, "hexkv_attend")
        return out


class StepWorkLists:
    """The work lists of consecutive decode steps, planned once on the host
    and kept in one device buffer.

    Step t attends ``lens[b] + t + 1`` keys per row (``+ t`` without
    ``kv_new``), for t < ``steps``; each step is planned with its own chunk
    (``partition`` 0: the library's choice for that step, else the given
    one) and, with ``single_launch``, for the device's XCDs.  ``self[t]`` is
    step t's ``WorkList``; ``chunks[t]`` its chunk and ``kernels[t]`` the
    kernel value it was planned with (``hexkv_attend_plan_kernel``: the
    row-block kernel for "auto" on large calls).  Nothing is planned or
    copied per step afterwards.
    """

    def __init__(self, p: _lib.AttendParams, lens: Sequence[int], steps: int, device,
                 single_launch: bool = True, partition: int = 0):
        if torch.cuda.is_current_stream_capturing():
            raise ValueError("StepWorkLists must be built before graph capture")
        lib = _lib.load()
        if len(lens) != p.batch:
            raise ValueError(f"{len(lens)} host lengths for a batch of {p.batch}")
        if steps < 1:
            raise ValueError("at least one step")
        q = _lib.AttendParams.from_buffer_copy(p)
        q.work_items_dev, q.work_parts_dev, q.lengths_out_dev = None, None, None
        q.work_xcds = _plan_xcds(q, device, single_launch)
        extra = 1 if q.kv_new else 0
        self.lens = [int(n) for n in lens]
        q.max_seqlen = max(self.lens, default=0) + steps - 1 + extra
        c_lens = (ctypes.c_int32 * len(self.lens))(*self.lens)
        n_segs = max(p.batch * p.q_heads, 1)  # head groups never outnumber query heads
        requested = q.kernel
        sizes, self.chunks, self.kernels = [], [], []
        for t in range(steps):
            q.seqlen_bias, q.kernel, q.partition = t, requested, 0
            q.kernel = _plan_kernel(q, c_lens)
            chunk, n, mp = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
            q.partition = int(partition)
            _lib.check(lib.hexkv_attend_plan_chunk(ctypes.byref(q), c_lens, ctypes.byref(chunk)),
                       "hexkv_attend_plan_chunk")
            q.partition = chunk.value
            _lib.check(lib.hexkv_attend_plan(ctypes.byref(q), c_lens, None, 0, None, 0, ctypes.byref(n),
                                             ctypes.byref(mp)), "hexkv_attend_plan")
            sizes.append((max(n.value, 1), mp.value))
            self.chunks.append(chunk.value)
            self.kernels.append(q.kernel)
        # one buffer: per step, its items (8 words each) then n_segs counts
        offsets, words = [], 0
        for n, _ in sizes:
            offsets.append(words)
            words += n * 8 + n_segs + (-(n * 8 + n_segs) % 4)  # keep every items block 16-byte aligned
        host = torch.zeros(words, dtype=torch.int32, pin_memory=True)
        base = host.data_ptr()
        for t, ((n, _), off) in enumerate(zip(sizes, offsets)):
            q.seqlen_bias, q.partition, q.kernel = t, self.chunks[t], self.kernels[t]
            got, mp = ctypes.c_int32(), ctypes.c_int32()
            _lib.check(lib.hexkv_attend_plan(ctypes.byref(q), c_lens, ctypes.c_void_p(base + off * 4), n,
                                             ctypes.c_void_p(base + (off + n * 8) * 4), n_segs, ctypes.byref(got),
                                             ctypes.byref(mp)), "hexkv_attend_plan")
        self.device_buffer = host.to(device)
        self.lists = [WorkList(self.device_buffer[off:off + n * 8].view(n, 8),
                               self.device_buffer[off + n * 8:off + n * 8 + n_segs], n, mp, q.work_xcds, k)
                      for (n, mp), off, k in zip(sizes, offsets, self.kernels)]
        self.steps, self.xcds = steps, q.work_xcds
        self.max_parts = max(mp for _, mp in sizes)
        self.max_seqlen = q.max_seqlen

    def __len__(self) -> int:
        return self.steps

    def __getitem__(self, t: int) -> WorkList:
        return self.lists[t]


class DecodeStepGraph:
    """One decode step's fused append + attend over every layer as a
    captured HIP graph, replayed per step.

    ``positions`` (device int32 ``[B]``) holds each sequence's cached length.
    A replay writes ``kv_new[l]`` at each sequence's position in every
    layer's cache, attends the keys up to and including it with ``q[l]``
    into ``out[l]``, and advances ``positions`` by one, all inside the graph:
    the host issues one launch per step instead of one or two per layer.
    ``max_seqlen`` bounds the attended length over every replay.  This is the
    graph-captured decode step of hexgen_core's generation loop
    (hexgen/hexgen_core/generation.py:354-443) restricted to the KV path.

    Without ``lens`` the attention runs the library's uniform partitions over
    the lengths in ``positions`` (one graph, positions advanced by a small
    kernel after the last layer).  With ``lens``, the host values of
    ``positions`` at the first replay, every step's work list is planned up
    front (``StepWorkLists``, with ``single_launch`` for the device's XCDs)
    and each step is its own captured graph over its own list, in which the
    last layer's attention kernel also stores the new lengths to
    ``positions``: a replay does no host planning, no copy and no extra
    launch.  Replay k then attends ``lens + k + 1`` keys, and ``max_seqlen``
    (which sets how many steps are captured) should be tight.  ``step``
    counts the replays; ``partition`` sets the positions per partition (grid)
    or per item (work lists); 0 leaves it to the library.

    The kernels must have run once eagerly in this process before capture
    (code objects load on first launch).  Graph nodes hold the tensors'
    addresses: the tensors must stay alive, and be updated in place, for as
    long as the graphs are replayed.
    """

    def __init__(self, q_layers: TensorList, cache_layers: TensorList, out_layers: TensorList,
                 kv_new_layers: TensorList, positions: torch.Tensor, max_seqlen: int,
                 softmax_scale: Optional[float] = None, kernel: str = "auto",
                 lens: Optional[Sequence[int]] = None, partition: int = 0, single_launch: bool = True):
        self.q, self.cache = _as_layers(q_layers), _as_layers(cache_layers)
        self.out, self.kv_new = _as_layers(out_layers), _as_layers(kv_new_layers)
        if not (len(self.q) == len(self.cache) == len(self.out) == len(self.kv_new)) or not self.q:
            raise ValueError("one q, cache, out and kv_new tensor per layer")
        _require_device(positions)
        if positions.dtype != torch.int32 or not positions.is_contiguous():
            raise ValueError("positions must be a contiguous int32 device tensor")
        self.positions, self.max_seqlen = positions, int(max_seqlen)
        self.plan = AttendPlan(self.q[0], self.cache[0], self.out[0], max_seqlens=[self.max_seqlen],
                               seqlens=positions, kv_new=self.kv_new[0], softmax_scale=softmax_scale,
                               kernel=kernel, partition=partition)
        # Every layer is checked before anything is captured.
        for l in range(len(self.q)):
            self.plan.check(self.q[l], self.cache[l], self.out[l], self.kv_new[l])
        self.lists = None
        self.step = 0
        if lens is None:
            self.graphs = [torch.cuda.CUDAGraph()]
            with torch.cuda.graph(self.graphs[0]):
                for l in range(len(self.q)):
                    self.plan(self.q[l], self.cache[l], self.out[l], self.kv_new[l], 0, self.max_seqlen)
                self.positions.add_(1)
            return
        steps = self.max_seqlen - max([int(n) for n in lens], default=0)
        if steps < 1:
            raise ValueError(f"max_seqlen {max_seqlen} leaves no step for lengths up to {max(lens)}")
        self.lists = StepWorkLists(self.plan.params, lens, steps, positions.device, single_launch, partition)
        self.plan.reserve(self.lists.lists)
        self.graphs = []
        pool = None
        last = len(self.q) - 1
        for t in range(steps):
            self.plan.fix_work_list(self.lists[t])
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool=pool):
                for l in range(len(self.q)):
                    self.plan(self.q[l], self.cache[l], self.out[l], self.kv_new[l], 0, self.max_seqlen,
                              lengths_out=self.positions if l == last else None)
            pool = graph.pool()
            self.graphs.append(graph)

    def replay(self) -> None:
        if self.lists is None:
            self.graphs[0].replay()
        else:
            if self.step >= len(self.graphs):
                raise RuntimeError(f"work lists captured for replays 0..{len(self.graphs) - 1}, "
                                   f"asked for {self.step}")
            self.graphs[self.step].replay()
        self.step += 1

    def restart(self) -> None:
        """Make the next replay replay 0 again (a new decode over the same
        lengths); the caller restores ``positions`` and the caches."""
        self.step = 0


class FtDecodeStepGraph:
    """``DecodeStepGraph`` over FasterTransformer caches: one HIP graph per
    decode step holding every layer's ``ft_attend`` (rotary, append at
    ``positions``, attention over ``[0, positions]``) and the advance of
    ``positions`` by one.  This is the layout the reference's CUDA-graph
    decode captures (hexgen/hexgen_core/generation.py:354-443 requires
    ``fused_ft_kernel``).  ``max_position`` bounds every position over every
    replay and must stay below the caches' capacity.

    As with ``DecodeStepGraph``, the kernels must have run once eagerly
    before capture, and every captured tensor must stay alive and be updated
    in place while the graph is replayed.
    """

    def __init__(self, q_layers: TensorList, k_cache_layers: TensorList, v_cache_layers: TensorList,
                 out_layers: TensorList, k_new_layers: TensorList, v_new_layers: TensorList,
                 positions: torch.Tensor, max_position: int, rotary_dim: int = 0,
                 rotary_base: float = 10000.0, rotary_neox: bool = True,
                 softmax_scale: Optional[float] = None):
        self.q, self.out = _as_layers(q_layers), _as_layers(out_layers)
        self.k_cache, self.v_cache = _as_layers(k_cache_layers), _as_layers(v_cache_layers)
        self.k_new, self.v_new = _as_layers(k_new_layers), _as_layers(v_new_layers)
        n = len(self.q)
        if not n or any(len(x) != n for x in (self.out, self.k_cache, self.v_cache, self.k_new, self.v_new)):
            raise ValueError("one q, out, K cache, V cache, k_new and v_new tensor per layer")
        _require_device(positions)
        if positions.dtype != torch.int32 or not positions.is_contiguous():
            raise ValueError("positions must be a contiguous int32 device tensor")
        self.positions, self.max_position = positions, int(max_position)
        need = ft_attend_workspace_bytes(self.q[0], self.k_cache[0], self.v_cache[0], self.max_position)
        self.workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=self.q[0].device)
        self.args = dict(max_position=self.max_position, positions=positions, rotary_dim=rotary_dim,
                         rotary_base=rotary_base, rotary_neox=rotary_neox, softmax_scale=softmax_scale,
                         workspace=self.workspace)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            for l in range(n):
                ft_attend(self.q[l], self.k_new[l], self.v_new[l], self.k_cache[l], self.v_cache[l],
                          out=self.out[l], **self.args)
            self.positions.add_(1)

    def replay(self) -> None:
        self.graph.replay()
