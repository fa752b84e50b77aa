"""Legacy KV-cache formats of HexGen's earlier disaggregation scripts, on the
hexkv library.

Three layouts and their wire messages, with the names, arguments and results
of the reference modules:

* the flat KV packet: every layer flattened and concatenated, shipped with its
  shapes (hexgen/llama/kv_cache_communication.py);
* zero-padded request batching: requests' caches padded to the longest and
  stacked along the batch (hexgen/llama/kv_cache_batch.py);
* tensor-parallel head concatenation: shards of the KV heads joined along
  dim 3 (hexgen/llama/tensor_parallel_dim_concat.py).

The byte movement of each is one ``hexkv_flat_concat`` / ``hexkv_batch_pad``
/ ``hexkv_head_concat`` call over every layer: strided byte rows moved by a
HIP kernel, on the current stream.  Device tensors only; a tensor whose
layout the block description cannot express is made contiguous first.

Zero-padded batches attend padded zeros as real keys when decoded with the
longest length (kv_cache_management.py:56-59 decodes with max(seqlen_og));
``batched_lengths`` gives each batched sequence's true length, which the
hexkv decode path (per-sequence ``seqlens``) uses instead.
"""
from __future__ import annotations

import array
import ctypes
import functools
import itertools
import math
from typing import Dict, List, Optional, Sequence, Tuple

import torch
import torch.distributed as dist

from . import _lib
from .ops import _require_device, _stream

# --------------------------------------------------------------- blocks ---


@functools.lru_cache(maxsize=4096)
def _layout(shape: Tuple[int, ...], stride: Tuple[int, ...], elem: int,
            split: Optional[int]) -> Optional[Tuple[int, int, int, int, int]]:
    """(width, height, depth, row_pitch, slice_pitch) in bytes of a tensor of
    this shape and stride, or None; see ``_as_block``.  Cached: the layers of
    one call usually share their shape and stride."""
    nd = len(shape)
    if split is None:
        split, expect = nd, 1
        while split > 0 and (shape[split - 1] == 1 or stride[split - 1] == expect):
            expect *= shape[split - 1]
            split -= 1
    expect = 1
    for d in range(nd - 1, split - 1, -1):
        if shape[d] != 1 and stride[d] != expect:
            return None
        expect *= shape[d]
    width = math.prod(shape[split:]) * elem
    outer = [(shape[d], stride[d]) for d in range(split) if shape[d] != 1]
    merged: List[Tuple[int, int]] = []
    for size, st in outer:  # fold a dim into the previous one when they are contiguous
        if merged and merged[-1][1] == size * st:
            merged[-1] = (merged[-1][0] * size, st)
        else:
            merged.append((size, st))
    if len(merged) > 2:
        return None
    while len(merged) < 2:
        merged.insert(0, (1, 0))
    (depth, s_pitch), (height, r_pitch) = merged
    if 0 in shape:
        depth, height, width = 0, 0, 0
    return width, height, depth, r_pitch * elem, s_pitch * elem


def _block_fields(t: torch.Tensor, split: Optional[int] = None,
                  shape: Optional[Tuple[int, ...]] = None) -> Optional[Tuple[int, ...]]:
    """``hexkv_block`` fields (data, width, height, depth, row_pitch,
    slice_pitch) of ``t``, or None; see ``_as_block``.  ``shape``: the
    caller's ``tuple(t.shape)``, when it has it already."""
    lay = _layout(tuple(t.shape) if shape is None else shape, t.stride(), t.element_size(), split)
    return None if lay is None else (t.data_ptr(), *lay)


def _as_block(t: torch.Tensor, split: Optional[int] = None) -> Optional[_lib.Block]:
    """Describe ``t`` as a hexkv block: rows are the dims from ``split`` on
    (contiguous), indexed by the dims before it collapsed into at most two
    strided levels (slices, rows).  ``split`` defaults to the start of the
    longest contiguous trailing run.  Returns None when the layout needs
    more levels or the row dims are not contiguous."""
    fields = _block_fields(t, split)
    return None if fields is None else _lib.Block(*fields)


def _block(t: torch.Tensor, split: Optional[int] = None,
           shape: Optional[Tuple[int, ...]] = None) -> Tuple[Tuple[int, ...], torch.Tensor]:
    """(block fields, tensor they describe): the tensor itself, or a
    contiguous copy when its layout has no block description."""
    fields = _block_fields(t, split, shape)
    if fields is None:
        t = t.contiguous()
        fields = _block_fields(t, split)
    return fields, t


def _block_array(fields: Sequence[Tuple[int, ...]]):
    """A ``hexkv_block`` array of these fields, built in one allocation (the
    struct is six 8-byte words: a pointer and five int64).  The words go
    through ``array.array``, which converts them in C: ctypes' own array
    constructor from a list took most of the host time of a 22-layer,
    4-shard head concatenation (~50 us for its 528 words)."""
    words = array.array("q", list(itertools.chain.from_iterable(fields)))
    # the ctypes view keeps `words` alive, and the cast keeps the view alive
    return ctypes.cast((ctypes.c_int64 * len(words)).from_buffer(words), ctypes.POINTER(_lib.Block))


def _one_dtype(tensors: Sequence[torch.Tensor], what: str) -> torch.dtype:
    if not tensors:
        raise ValueError(f"{what}: no tensors")
    _require_device(*tensors)
    dtype, device = tensors[0].dtype, tensors[0].device
    for t in tensors:
        if t.dtype != dtype or t.device != device:
            raise ValueError(f"{what}: tensors must share one dtype and device")
    return dtype


# ------------------------------------------------- flat packet (a + wire) ---


def flat_concat(tensors: Sequence[torch.Tensor], out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``torch.cat([t.flatten() for t in tensors])`` in one launch
    (kv_cache_communication.py:21-26): a 1-D tensor of every element, tensor
    by tensor in row-major order."""
    tensors = list(tensors)
    dtype = _one_dtype(tensors, "flat_concat")
    total = sum(t.numel() for t in tensors)
    if out is None:
        out = torch.empty(total, dtype=dtype, device=tensors[0].device)
    elif out.dtype != dtype or out.numel() != total or not out.is_contiguous():
        raise ValueError(f"flat_concat: out must be a contiguous {dtype} tensor of {total} elements")
    keep, blocks = [], []
    for t in tensors:
        b, t = _block(t)
        keep.append(t)
        blocks.append(b)
    rc = _lib.load().hexkv_flat_concat(_block_array(blocks), len(blocks), out.data_ptr(), _stream(out))
    _lib.check(rc, "hexkv_flat_concat")
    return out


def flat_views(flat: torch.Tensor, shapes: Sequence[Sequence[int]]) -> Dict[int, torch.Tensor]:
    """The receiver's layer dict: consecutive views of the flat packet
    reshaped to each shape (kv_cache_communication.py:50-57)."""
    out, off = {}, 0
    for i, shape in enumerate(shapes):
        n = math.prod(shape)
        out[i] = flat[off:off + n].view(tuple(shape))
        off += n
    if off != flat.numel():
        raise ValueError(f"shapes hold {off} elements, the packet {flat.numel()}")
    return out


def _send(t: torch.Tensor, dst: int, group) -> None:
    # Gloo moves host tensors only: stage device tensors through host memory.
    if dist.get_backend(group) == "gloo" and t.is_cuda:
        t = t.cpu()
    dist.send(t, dst=dst, group=group)


def _recv(shape, dtype, src: int, group, device) -> torch.Tensor:
    if dist.get_backend(group) == "gloo":
        t = torch.empty(shape, dtype=dtype)
        dist.recv(t, src=src, group=group)
        return t.to(device)
    t = torch.empty(shape, dtype=dtype, device=device)
    dist.recv(t, src=src, group=group)
    return t


def _device(device) -> torch.device:
    return torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)


def send_logits_with_seqlen_og(logits: torch.Tensor, seqlen_og: int, dst: int, group=None) -> None:
    """kv_cache_communication.py:5-8: int64 ``[seqlen_og, *logits.shape]``,
    then the logits."""
    meta = torch.tensor([seqlen_og] + [*logits.shape], dtype=torch.long, device=logits.device)
    _send(meta, dst, group)
    _send(logits.contiguous(), dst, group)


def recv_logits_with_seqlen_og(src: int, dim: int = 3, group=None, dtype=torch.float16,
                               device=None) -> Tuple[torch.Tensor, int]:
    """kv_cache_communication.py:10-18 (``dim`` = 1 + the logits' rank; the
    reference receives float16 logits)."""
    device = _device(device)
    meta = _recv((dim,), torch.long, src, group, device).tolist()
    logits = _recv(tuple(meta[1:]), dtype, src, group, device)
    return logits, int(meta[0])


def send_key_value_memory_dict(key_value_memory_dict: Dict[int, torch.Tensor], dst: int, group=None) -> None:
    """kv_cache_communication.py:20-32: the layer count, each shape's rank,
    the flattened shapes (int64), then the flat packet built by one
    ``hexkv_flat_concat``."""
    tensors = list(key_value_memory_dict.values())
    shapes = [tuple(t.shape) for t in tensors]
    flat = flat_concat(tensors)
    device = flat.device
    _send(torch.tensor([len(tensors)], dtype=torch.long, device=device), dst, group)
    _send(torch.tensor([len(s) for s in shapes], dtype=torch.long, device=device), dst, group)
    _send(torch.tensor([d for s in shapes for d in s], dtype=torch.long, device=device), dst, group)
    _send(flat, dst, group)


def recv_key_value_memory_dict(src: int, group=None, dtype=torch.float16, device=None) -> Dict[int, torch.Tensor]:
    """kv_cache_communication.py:34-58: the layer dict as views of one
    received flat buffer, keyed 0..n-1 (the reference receives float16)."""
    device = _device(device)
    n = int(_recv((1,), torch.long, src, group, device).item())
    ranks = _recv((n,), torch.long, src, group, device).tolist()
    flat_shapes = _recv((sum(ranks),), torch.long, src, group, device).tolist()
    shapes, off = [], 0
    for r in ranks:
        shapes.append(tuple(flat_shapes[off:off + r]))
        off += r
    flat = _recv((sum(math.prod(s) for s in shapes),), dtype, src, group, device)
    return flat_views(flat, shapes)


def kv_cache_communication_send(logits, seqlen_og, key_value_memory_dict, dst, group=None) -> None:
    """kv_cache_communication.py:60-62."""
    send_logits_with_seqlen_og(logits, seqlen_og, dst, group)
    send_key_value_memory_dict(key_value_memory_dict, dst, group)


def kv_cache_communication_recv(src, group=None, dtype=torch.float16, device=None):
    """kv_cache_communication.py:64-67: ``(logits, seqlen_og, kv dict)``."""
    logits, seqlen_og = recv_logits_with_seqlen_og(src, group=group, dtype=dtype, device=device)
    return logits, seqlen_og, recv_key_value_memory_dict(src, group, dtype, device)


# ------------------------------------------------------ zero-pad batching ---


def batch_key_value_memory_dicts(kv_memory_dicts_list: Sequence[Dict[int, torch.Tensor]],
                                 max_rows: Optional[int] = None) -> Dict[int, torch.Tensor]:
    """The KV half of batch_logits_and_key_value_memory_dict
    (kv_cache_batch.py:11-22): per key, each request's ``[b_i, S_i, ...]``
    zero-padded at the end of dim 1 to ``max_rows`` (default max S_i) and
    stacked along dim 0 -- every layer in one ``hexkv_batch_pad``.  The
    result's tensors are views of one allocation, one per key."""
    dicts = list(kv_memory_dicts_list)
    if not dicts:
        raise ValueError("no requests to batch")
    keys = list(dicts[0].keys())
    if not keys:
        return {}
    first = [d[keys[0]] for d in dicts]
    grid = [[d[key] for d in dicts] for key in keys]  # [key][request]
    dtype = _one_dtype([t for row in grid for t in row], "batch_key_value_memory_dicts")
    if any(t.dim() < 2 for t in first):
        raise ValueError("cache tensors must be [batch, positions, ...]")
    shapes = [[tuple(t.shape) for t in row] for row in grid]
    rest = shapes[0][0][2:]
    heads, ragged = [sh[:2] for sh in shapes[0]], False
    for key, row in zip(keys, shapes):
        for i, shape in enumerate(row):
            if len(shape) < 2 or shape[2:] != rest:
                raise ValueError(f"request {i} layer {key}: shape {shape} does not batch with "
                                 f"rows of shape {rest}")
            ragged = ragged or shape[:2] != heads[i]
    if ragged:
        # a request's sizes differ between layers: each key is padded to its
        # own longest request (kv_cache_batch.py:14), one launch per key
        out = {}
        for key in keys:
            out.update({key: batch_key_value_memory_dicts([{key: d[key]} for d in dicts], max_rows)[key]})
        return out
    longest = max(sh[1] for sh in shapes[0])
    max_rows = longest if max_rows is None else int(max_rows)
    seqs = sum(sh[0] for sh in shapes[0])
    out = torch.empty((len(keys), seqs, max_rows, *rest), dtype=dtype, device=first[0].device)
    views = out.unbind(0)
    keep, blocks = [], []
    elem = first[0].element_size()
    width = math.prod(rest) * elem
    # rows (dims 2+) are contiguous when every dim of size > 1 has its
    # contiguous stride
    row_dims = [d for d in range(len(rest)) if rest[d] != 1]
    row_strides = tuple(math.prod(rest[d + 1:]) for d in row_dims)
    for row, row_shapes in zip(grid, shapes):
        for t, shape in zip(row, row_shapes):
            st = t.stride()
            if tuple(st[2 + d] for d in row_dims) != row_strides and 0 not in shape:
                t = t.contiguous()
                st = t.stride()
            # depth = the request's sequences, height = its positions
            b, n = shape[0], shape[1]
            blocks.append((t.data_ptr() if b * n else 0, width, n, b, st[1] * elem, st[0] * elem))
            keep.append(t)
    dst = (ctypes.c_void_p * len(keys))(*[v.data_ptr() for v in views])
    rc = _lib.load().hexkv_batch_pad(_block_array(blocks), len(keys), len(dicts), dst, max_rows, _stream(out))
    _lib.check(rc, "hexkv_batch_pad")
    return dict(zip(keys, views))


def batch_logits_and_key_value_memory_dict(logits_list: Sequence[torch.Tensor],
                                           kv_memory_dicts_list: Sequence[Dict[int, torch.Tensor]]):
    """kv_cache_batch.py:4-28: ``(logits concatenated along dim 0, batched
    KV dict)``.  Logits of equal trailing shape are concatenated by one
    ``hexkv_flat_concat``."""
    logits_list = list(logits_list)
    if not logits_list:
        raise ValueError("no logits to batch")
    tail = tuple(logits_list[0].shape[1:])
    if any(tuple(l.shape[1:]) != tail for l in logits_list):
        raise ValueError("logits must agree in every dim but the first")
    rows = sum(l.shape[0] for l in logits_list)
    logits = flat_concat(logits_list).view(rows, *tail)
    return logits, batch_key_value_memory_dicts(kv_memory_dicts_list)


def batched_lengths(kv_memory_dicts_list: Sequence[Dict[int, torch.Tensor]]) -> List[int]:
    """True length of every sequence of a zero-padded batch, in batch order:
    request i contributes b_i copies of its S_i."""
    out = []
    for d in kv_memory_dicts_list:
        t = next(iter(d.values()))
        out.extend([int(t.shape[1])] * int(t.shape[0]))
    return out


# -------------------------------------------------------- TP head concat ---


def concat_dicts(list_of_dicts: Sequence[Dict[int, torch.Tensor]], dim: int = 3) -> Dict[int, torch.Tensor]:
    """tensor_parallel_dim_concat.py:9-19: per key, the shards concatenated
    along ``dim`` (3 = the KV heads of ``[B, S, 2, H, D]``), every key in one
    ``hexkv_head_concat``: one row per index of the dims before ``dim``,
    shard j's slice of the dims from ``dim`` on at its column."""
    dicts = list(list_of_dicts)
    if not dicts:
        raise ValueError("no shards to concatenate")
    keys = list(dicts[0].keys())
    if not keys:
        return {}
    ref = dicts[0][keys[0]]
    nd = ref.dim()
    if not -nd <= dim < nd:
        raise ValueError(f"dim {dim} out of range for {nd}-d tensors")
    dim %= nd
    grid = [[d[key] for d in dicts] for key in keys]  # [key][shard]
    dtype = _one_dtype([t for row in grid for t in row], "concat_dicts")
    shapes = [[tuple(t.shape) for t in row] for row in grid]
    for key, row in zip(keys, shapes):
        s0 = row[0]
        for sh in row:
            if len(sh) != nd or sh[:dim] != s0[:dim] or sh[dim + 1:] != s0[dim + 1:]:
                raise ValueError(f"key {key}: shard shapes {row} do not concatenate along dim {dim}")
    if any(row != shapes[0] for row in shapes):
        # layers of different shapes: one launch per key
        return {key: _concat_one(row, dim) for key, row in zip(keys, grid)}
    s0 = shapes[0][0]
    out = torch.empty((len(keys), *s0[:dim], sum(sh[dim] for sh in shapes[0]), *s0[dim + 1:]),
                      dtype=dtype, device=ref.device)
    views = out.unbind(0)
    _head_concat(grid, views, dim, shapes)
    return dict(zip(keys, views))


def _concat_one(shards: Sequence[torch.Tensor], dim: int) -> torch.Tensor:
    s0 = shards[0].shape
    out = torch.empty((*s0[:dim], sum(t.shape[dim] for t in shards), *s0[dim + 1:]), dtype=shards[0].dtype,
                      device=shards[0].device)
    _head_concat([list(shards)], [out], dim)
    return out


def _head_concat(layers: Sequence[Sequence[torch.Tensor]], outs: Sequence[torch.Tensor], dim: int,
                 shapes: Optional[Sequence[Sequence[Tuple[int, ...]]]] = None) -> None:
    """One hexkv_head_concat over every layer: rows are the indices of the
    dims before ``dim`` (however each shard folds them), a shard's row its
    slice of the dims from ``dim`` on.  ``shapes``: the shards' shapes as
    tuples, when the caller has them."""
    keep, blocks = [], []
    for i, shards in enumerate(layers):
        for j, t in enumerate(shards):
            sh = tuple(t.shape) if shapes is None else shapes[i][j]
            if 0 in sh:  # no heads in this shard, or no rows at all
                b = (0, math.prod(sh[dim:]) * t.element_size(), math.prod(sh[:dim]), 1, 0, 0)
            else:
                b, t = _block(t, split=dim, shape=sh)
            keep.append(t)
            blocks.append(b)
    dst = (ctypes.c_void_p * len(layers))(*[o.data_ptr() for o in outs])
    rc = _lib.load().hexkv_head_concat(_block_array(blocks), len(layers), len(layers[0]), dst, _stream(outs[0]))
    _lib.check(rc, "hexkv_head_concat")


def tensor_parallel_dim_concat(logits_list, seqlen_og_list, key_value_memory_dict_list):
    """tensor_parallel_dim_concat.py:3-7: the first shard's logits and
    seqlen_og, and the shards' KV dicts joined along the heads."""
    return logits_list[0], seqlen_og_list[0], concat_dicts(key_value_memory_dict_list)
