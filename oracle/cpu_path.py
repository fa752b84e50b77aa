"""The reference's PyTorch operations for the KV path, on CPU tensors -- the
timed CPU baseline.  TEST/BENCH INFRASTRUCTURE ONLY (never the product path).

* ``pack``    hexgen2/model.py:81  ``t[:, :L].contiguous()`` per layer and
              sequence, concatenated per layer (batch-1 packets laid end to end)
* ``unpack``  hexgen2/model.py:105-107  ``torch.empty`` + ``copy_`` per layer
* ``append``  hexgen/hexgen_core/modules/mha.py:286  slice assignment
* ``attend``  hexgen/hexgen_core/modules/mha.py:219-244  CrossAttention: GQA
              repeat, einsum scores, softmax in ``v.dtype``, einsum output;
              one call per sequence because lengths are ragged
"""
from __future__ import annotations

import math
from typing import Sequence

import torch


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
