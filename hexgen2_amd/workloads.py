"""Synthetic KV-path workloads and their algorithmic byte counts.

Each workload is a model's KV geometry plus a seeded batch of ragged prompt
lengths.  Byte counts are what the data path must move at minimum (live rows
only, each byte once):

* pack   = layers * sum(L_b) * row   read  + the same written
* unpack = the same again, so pack+unpack = 4 * layers * sum(L_b) * row
* decode step t (all layers) = layers * [ sum_b (L_b + t + 1) * row   K/V read
                                          + 2 * B * row                 append: kv_new read + row written
                                          + 2 * B * Hq * D * elem ]     q read + output written
  where row = 2 * Hkv * D * elem.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List

import torch


@dataclass
class KVWorkload:
    name: str
    layers: int
    kv_heads: int
    q_heads: int
    head_dim: int
    dtype: torch.dtype
    batch: int
    len_lo: int
    len_hi: int
    decode_steps: int
    capacity: int = 0  # 0: max prompt length + decode steps
    seed: int = 0
    lens: List[int] = field(default_factory=list)

    def __post_init__(self):
        if not self.lens:
            g = torch.Generator().manual_seed(self.seed)
            if self.len_lo == self.len_hi:
                self.lens = [self.len_lo] * self.batch
            else:
                self.lens = torch.randint(self.len_lo, self.len_hi + 1, (self.batch,), generator=g).tolist()
        if not self.capacity:
            self.capacity = max(self.lens) + self.decode_steps

    @property
    def elem(self) -> int:
        return torch.empty((), dtype=self.dtype).element_size()

    @property
    def row_bytes(self) -> int:
        return 2 * self.kv_heads * self.head_dim * self.elem

    @property
    def live_rows(self) -> int:
        return sum(self.lens)

    def pack_bytes(self) -> int:
        """Algorithmic bytes of one pack (= one unpack) over all layers."""
        return 2 * self.layers * self.live_rows * self.row_bytes

    def pack_unpack_bytes(self) -> int:
        return 2 * self.pack_bytes()

    def attend_bytes(self, step: int) -> int:
        """Bytes of one layer's fused append+attend at decode step ``step``."""
        kv_read = (self.live_rows + self.batch * (step + 1)) * self.row_bytes
        append = 2 * self.batch * self.row_bytes
        q_out = 2 * self.batch * self.q_heads * self.head_dim * self.elem
        # the appended row is read from kv_new, not from the cache: count it once
        return kv_read - self.batch * self.row_bytes + append + q_out

    def decode_bytes(self, steps=None) -> int:
        """Bytes of ``steps`` decode steps over all layers."""
        steps = self.decode_steps if steps is None else steps
        return self.layers * sum(self.attend_bytes(t) for t in range(steps))

    def describe(self) -> dict:
        return {"workload": self.name, "layers": self.layers, "kv_heads": self.kv_heads,
                "q_heads": self.q_heads, "head_dim": self.head_dim, "dtype": str(self.dtype).split(".")[-1],
                "batch": self.batch, "prompt_lengths": f"U[{self.len_lo},{self.len_hi}] seed {self.seed}"
                if self.len_lo != self.len_hi else str(self.len_lo),
                "sum_prompt_lengths": self.live_rows, "capacity": self.capacity,
                "decode_steps": self.decode_steps}


def workload(name: str, **overrides) -> KVWorkload:
    """The configurations the path is measured and checked on."""
    table = {
        "tiny-llama": dict(layers=2, kv_heads=4, q_heads=4, head_dim=16, dtype=torch.float32,
                           batch=1, len_lo=16, len_hi=16, decode_steps=7, capacity=24),
        "tinyllama-1.1b": dict(layers=22, kv_heads=4, q_heads=32, head_dim=64, dtype=torch.float16,
                               batch=1, len_lo=512, len_hi=512, decode_steps=128, capacity=2048),
        "llama2-7b": dict(layers=32, kv_heads=32, q_heads=32, head_dim=128, dtype=torch.float16,
                          batch=8, len_lo=256, len_hi=2048, decode_steps=64, capacity=4096),
        "llama2-70b-tp8": dict(layers=80, kv_heads=1, q_heads=8, head_dim=128, dtype=torch.bfloat16,
                               batch=32, len_lo=512, len_hi=4096, decode_steps=32),
        "llama3-8b": dict(layers=32, kv_heads=8, q_heads=32, head_dim=128, dtype=torch.bfloat16,
                          batch=64, len_lo=128, len_hi=8192, decode_steps=256),
    }
    if name not in table:
        raise KeyError(f"unknown workload {name!r}; known: {sorted(table)}")
    args = dict(table[name])
    args.update(overrides)
    return KVWorkload(name=name, **args)


WORKLOADS = ("tiny-llama", "tinyllama-1.1b", "llama2-7b", "llama2-70b-tp8", "llama3-8b")
