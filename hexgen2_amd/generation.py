"""Cache-state type of the decode path.

Same fields and defaults as hexgen_core's ``InferenceParams``
(hexgen/hexgen_core/generation.py:20-30) and the pilot's ``CacheState``
(hexgen2/model.py:11-19), so callers written against either keep working.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import torch


@dataclass
class InferenceParams:
    """Per-request KV-cache state.

    ``key_value_memory_dict`` maps layer index -> cache tensor
    ``[max_batch_size, max_sequence_len, 2, kv_heads, head_dim]``, or with
    ``fused_ft_kernel`` the FasterTransformer pair ``(K [B, H, D/pack, S,
    pack], V [B, H, S, D])``; ``sequence_len_offset`` is the number of
    positions already cached (the append position of the next token);
    ``lengths_per_sample`` (int32, device), when set, gives each sequence's
    own position (its cached length) in a ragged decode batch, on the FT path
    and on the standard layout alike; ``sequence_len_offset`` then bounds
    every sample's position.
    """
    max_sequence_len: int
    max_batch_size: int = 1
    sequence_len_offset: int = 0
    batch_size_offset: int = 0
    key_value_memory_dict: dict = field(default_factory=dict)
    fused_ft_kernel: bool = False
    lengths_per_sample: Optional[torch.Tensor] = None


# hexgen2/model.py:11-19 names the same record CacheState.
CacheState = InferenceParams
