"""The reference's PyTorch operations for the KV path, on CPU tensors -- the
timed CPU baseline.  TEST/BENCH INFRASTRUCTURE ONLY (never the product path).

* ``pack``    hexgen2/model.py:81  ``t[:, :L].contiguous()`` per layer and
              sequence, concatenated per layer (batch-1 packets laid end to end)
* ``unpack``  hexgen2/model.py:105-107  ``torch.empty`` + ``copy_`` per layer
* ``append``  hexgen/hexgen_core/modules/mha.py:286  slice assignment
* ``attend``  hexgen/hexgen_core/modules/mha.py:219-244  CrossAttention: GQA
              repeat, einsum scores, softmax in ``v.dtype``, einsum output;
              one call per sequence because lengths are ragged
* ``flat_concat``  hexgen/llama/kv_cache_communication.py:21-26  every
              tensor flattened, ``torch.cat``
* ``batch_pad``    hexgen/llama/kv_cache_batch.py:11-26  per key, ``F.pad``
              of dim 1 to the longest request, ``torch.cat`` along dim 0
* ``concat_dicts`` hexgen/llama/tensor_parallel_dim_concat.py:9-19  per key,
              ``torch.cat`` along ``dim``
* ``ft_store``     hexgen/hexgen_core/modules/mha.py:301-306  the FT branch's
              prefill write: K rearranged to ``b h d s packsize``, V to
              ``b h s d``, assigned into the caches
"""
from __future__ import annotations

import math
from typing import Sequence

import torch
import torch.nn.functional as F


def pack(layers: Sequence[torch.Tensor], lens: Sequence[int]) -> list:
    return [torch.cat([t[b:b + 1, :n].contiguous()[0] for b, n in enumerate(lens)], dim=0)
            for t in layers]


def unpack(packed: Sequence[torch.Tensor], capacity: int, lens: Sequence[int]) -> list:
    out = []
    for live in packed:
        full = torch.empty((len(lens), capacity, *live.shape[1:]), dtype=live.dtype)
        start = 0
        for b, n in enumerate(lens):
            full[b:b + 1, :n].copy_(live[start:start + n])
            start += n
        out.append(full)
    return out


def append(cache: torch.Tensor, kv: torch.Tensor, positions: Sequence[int]) -> None:
    for b, pos in enumerate(positions):
        cache[b:b + 1, pos:pos + 1, ...] = kv[b:b + 1]


def attend(q: torch.Tensor, cache: torch.Tensor, lens: Sequence[int], softmax_scale=None) -> torch.Tensor:
    """q [B, 1, Hq, D], cache [B, S, 2, Hkv, D] -> [B, 1, Hq, D]."""
    outs = []
    for b, n in enumerate(lens):
        qb, kv = q[b:b + 1], cache[b:b + 1, :n]
        if kv.shape[3] != qb.shape[2]:
            kv = kv.repeat_interleave(qb.shape[2] // kv.shape[3], dim=3)
        k, v = kv.unbind(dim=2)
        scale = softmax_scale or 1.0 / math.sqrt(qb.shape[-1])
        scores = torch.einsum("bthd,bshd->bhts", qb, k * scale)
        attention = torch.softmax(scores, dim=-1, dtype=v.dtype)
        outs.append(torch.einsum("bhts,bshd->bthd", attention, v))
    return torch.cat(outs, dim=0)


def flat_concat(tensors: Sequence[torch.Tensor]) -> torch.Tensor:
    return torch.cat([t.flatten() for t in tensors])


def batch_pad(dicts: Sequence[dict]) -> dict:
    out = {}
    for key in dicts[0]:
        longest = max(d[key].size(1) for d in dicts)
        parts = []
        for d in dicts:
            t = d[key]
            pad = longest - t.size(1)
            parts.append(F.pad(t, (0, 0, 0, 0, 0, 0, 0, pad), "constant", 0) if pad > 0 else t)
        out[key] = torch.cat(parts, dim=0)
    return out


def concat_dicts(dicts: Sequence[dict], dim: int = 3) -> dict:
    return {key: torch.cat([d[key] for d in dicts], dim=dim) for key in dicts[0]}


def ft_store(kv: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor) -> None:
    """kv [B, S, 2, H, D] into k_cache [B, H, D/pack, capacity, pack] and
    v_cache [B, H, capacity, D] at positions [0, S)."""
    b, s, _, h, d = kv.shape
    pack = k_cache.shape[-1]
    k_cache[:b, :, :, :s, :] = kv[:, :, 0].reshape(b, s, h, d // pack, pack).permute(0, 2, 3, 1, 4)
    v_cache[:b, :, :s, :] = kv[:, :, 1].permute(0, 2, 1, 3)
