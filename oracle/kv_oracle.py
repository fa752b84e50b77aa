"""CPU oracle of the KV-cache data path -- TEST INFRASTRUCTURE ONLY.

A plain numpy restatement of what the reference computes on this path.  Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import it, and only as the checker: the product path (``hexgen2_amd``)
never calls it and has no CPU fallback.

Functions and the reference code each one restates:

* ``pack``      hexgen2/model.py:78-81   live prefix of each layer's cache,
                                         generalised to ragged batches; layers
                                         concatenated in send order
                                         (hexgen2/transport.py:56-59)
* ``unpack``    hexgen2/model.py:101-108 scatter into a preallocated cache
* ``append``    hexgen/hexgen_core/modules/mha.py:276-288 (slice assignment,
                                         per-sequence offsets)
* ``attend``    hexgen/hexgen_core/modules/mha.py:209-244 (CrossAttention:
                                         GQA repeat :223-224, scale :231,
                                         causal mask :238-241, softmax :242)
                                         evaluated in float64
* ``packet_payload_bytes``  hexgen2/transport.py:37 (payload accounting)
* ``flat_concat`` / ``flat_split``  hexgen/llama/kv_cache_communication.py:
                                         21-26 / 50-57 (flat KV packet)
* ``batch_pad`` hexgen/llama/kv_cache_batch.py:11-22 (zero-pad + stack)
* ``concat_dim`` hexgen/llama/tensor_parallel_dim_concat.py:9-19 (TP heads)
* ``ft_layout`` / ``ft_unlayout``  hexgen/hexgen_core/modules/mha.py:296-298,
                                         301-305 (the FasterTransformer K/V
                                         layouts, rearrange patterns) and its
                                         inverse
* ``round_to``  rounding to float16 / bfloat16 / float32, nearest-even
* ``rotary``    the rotary embedding applied to q and k at the token's
                                         position on the FT path (mha.py:
                                         310-337 -> ft_attention, not vendored;
                                         GPT-NeoX halves or GPT-J pairs,
                                         angle pos * base^(-2j / rot_dim))
* ``ft_decode`` mha.py:310-337: rotate q and k (rounded to the data type),
                                         write k, v at each sequence's
                                         position, attend over [0, position]

Pinning (tests/test_oracle.py): pack/unpack/append against element-by-element
Python loops on small inputs, the round-trip and untouched-row invariants, and
the reference's recorded handoff byte counts (evidence/2026-10-19/
fabric-pilot.json); attend against closed forms (one key -> that value, equal
keys -> mean of values, a dominant key -> its value, group 1 == MHA), a
scalar-loop restatement on small shapes, and torch's
scaled_dot_product_attention in float64.  The legacy formats against the
library routines the reference calls (torch.cat, torch.nn.functional.pad with
the reference's pad tuple) and against their inverses (slicing a batch or a
concatenation back into its parts recovers them; padding is zero).  The FT
layouts against einops.rearrange with the reference's own patterns and
against their inverse; ``rotary`` against closed forms (position 0 and
rot_dim 0 are the identity, every pair keeps its norm, a 2-vector turns by
pos radians) and, for the GPT-NeoX form, against transformers' Llama
``apply_rotary_pos_emb``, with the GPT-J form tied to it by the pair
permutation; ``round_to`` against torch's casts; ``ft_decode`` without
rotation against ``append`` + ``attend``.  One detail of ``ft_decode`` is
parity unpinned: the point where the rotated q and k are rounded to the data
type (after the rotation, before the products; the rotated k is what the
cache keeps).  It follows FasterTransformer's published masked-attention
kernel, which ft_attention wraps, but no output of that extension exists to
check it against; its effect is one rounding of q and k (within the
attention tolerances either way).
"""
from __future__ import annotations

import math
from typing import Sequence

import numpy as np


def cu_lengths(lens: Sequence[int]) -> np.ndarray:
    """Prefix sums [0, L0, L0+L1, ...]: packed row offset of each sequence."""
    out = np.zeros(len(lens) + 1, dtype=np.int64)
    np.cumsum(np.asarray(lens, dtype=np.int64), out=out[1:])
    return out


def pack(caches: Sequence[np.ndarray], lens: Sequence[int]) -> np.ndarray:
    """caches: per layer [B, S, *row]; returns [n_layers, sum(lens), *row].

    Row ``cu[b] + s`` of layer l is ``caches[l][b, s]`` for s < lens[b].
    """
    layers = []
    for cache in caches:
        if len(lens) != cache.shape[0]:
            raise ValueError("one length per sequence")
        if any(n < 0 or n > cache.shape[1] for n in lens):
            raise ValueError("length outside [0, capacity]")
        # model.py:81 -- t[:, :L] per sequence, concatenated in batch order
        layers.append(np.concatenate([cache[b, :n] for b, n in enumerate(lens)], axis=0))
    return np.stack(layers, axis=0)


def unpack(packed: np.ndarray, caches: Sequence[np.ndarray], lens: Sequence[int]) -> list:
    """Returns copies of ``caches`` with rows [0, lens[b]) of every sequence
    replaced from ``packed``; all other rows unchanged."""
    cu = cu_lengths(lens)
    out = []
    for l, cache in enumerate(caches):
        cache = cache.copy()
        for b, n in enumerate(lens):
            # model.py:107 -- full[:, :L].copy_(live)
            cache[b, :n] = packed[l, cu[b]:cu[b] + n]
        out.append(cache)
    return out


def append(cache: np.ndarray, kv_new: np.ndarray, positions: Sequence[int]) -> np.ndarray:
    """Copy of ``cache`` [B, S, *row] with ``cache[b, positions[b]] = kv_new[b]``."""
    cache = cache.copy()
    for b, pos in enumerate(positions):
        if not 0 <= pos < cache.shape[1]:
            # mha.py:282 asserts sequence_end <= capacity
            raise ValueError("append position outside the cache")
        cache[b, pos] = kv_new[b].reshape(cache.shape[2:])
    return cache


def attend(q: np.ndarray, cache: np.ndarray, lens: Sequence[int], causal: bool = False,
           softmax_scale: float | None = None) -> np.ndarray:
    """Float64 attention of q [B, Sq, Hq, D] over cache [B, S, 2, Hkv, D].

    Sequence b attends keys [0, lens[b]); with ``causal`` query t of Sq sees
    keys [0, lens[b] - Sq + t + 1) (equal to CrossAttention's triangular mask
    when Sq == lens[b], the prefill case).  Returns [B, Sq, Hq, D] float64.
    """
    q = np.asarray(q, dtype=np.float64)
    cache = np.asarray(cache, dtype=np.float64)
    batch, sq, hq, d = q.shape
    hkv = cache.shape[3]
    g = hq // hkv
    scale = 1.0 / math.sqrt(d) if softmax_scale is None else softmax_scale
    out = np.zeros_like(q)
    for b in range(batch):
        n = int(lens[b])
        # mha.py:223-224 -- repeat "... hkv d -> ... (hkv g) d": q head h uses kv head h // g
        k = np.repeat(cache[b, :n, 0], g, axis=1)  # [n, Hq, D]
        v = np.repeat(cache[b, :n, 1], g, axis=1)
        scores = np.einsum("thd,shd->hts", q[b], k * scale)  # mha.py:231
        if causal:
            t_idx = np.arange(sq)[:, None]
            s_idx = np.arange(n)[None, :]
            scores = np.where(s_idx <= n - sq + t_idx, scores, -np.inf)
        scores = scores - scores.max(axis=-1, keepdims=True)
        p = np.exp(scores)
        p /= p.sum(axis=-1, keepdims=True)
        out[b] = np.einsum("hts,shd->thd", p, v)  # mha.py:244
    return out


def attend_loop(q, cache, lens, softmax_scale=None) -> np.ndarray:
    """Scalar-loop restatement of ``attend`` (non-causal) for tiny shapes."""
    batch, sq, hq, d = q.shape
    hkv = cache.shape[3]
    g = hq // hkv
    scale = 1.0 / math.sqrt(d) if softmax_scale is None else softmax_scale
    out = np.zeros((batch, sq, hq, d))
    for b in range(batch):
        for t in range(sq):
            for h in range(hq):
                kvh = h // g
                scores = []
                for s in range(int(lens[b])):
                    scores.append(sum(float(q[b, t, h, i]) * float(cache[b, s, 0, kvh, i])
                                      for i in range(d)) * scale)
                m = max(scores)
                w = [math.exp(x - m) for x in scores]
                z = sum(w)
                for i in range(d):
                    out[b, t, h, i] = sum(w[s] * float(cache[b, s, 1, kvh, i])
                                          for s in range(len(w))) / z
    return out


DTYPE_BYTES = {"torch.float16": 2, "torch.bfloat16": 2, "torch.float32": 4,
               "torch.float64": 8, "torch.int64": 8, "torch.int32": 4, "torch.int16": 2,
               "torch.int8": 1, "torch.uint8": 1, "torch.bool": 1}


def packet_payload_bytes(tensors: Sequence[tuple]) -> int:
    """Sum of prod(shape) * element size over (shape, dtype-name) pairs
    (transport.py:37)."""
    return sum(math.prod(shape) * DTYPE_BYTES[dtype] for shape, dtype in tensors)


def kv_packet_bytes(n_layers: int, prompt_len: int, kv_heads: int, head_dim: int,
                    elem_bytes: int) -> int:
    """Bytes of the pilot's KV packet: the int64 first token plus one
    [1, L, 2, Hkv, D] live slice per layer (run.py:147-148)."""
    row = 2 * kv_heads * head_dim * elem_bytes
    return 8 + n_layers * prompt_len * row


# ---------------------------------------------------------- legacy formats ---
# The earlier disaggregation scripts (hexgen/llama/) move the KV dict in three
# more layouts.  All three are element permutations (plus zero padding), so
# the restatements below work on arrays of any dtype, including integer views
# of float payloads.


def flat_concat(tensors: Sequence[np.ndarray]) -> np.ndarray:
    """The flat packet of send_key_value_memory_dict: every tensor flattened
    in row-major order and concatenated (kv_cache_communication.py:21-26)."""
    parts = [np.asarray(t).reshape(-1) for t in tensors]
    if not parts:
        return np.zeros(0)
    return np.concatenate(parts)


def flat_split(flat: np.ndarray, shapes: Sequence[tuple]) -> list:
    """The receiver's views of the flat packet (kv_cache_communication.py:
    50-57): consecutive slices reshaped to each shape."""
    out, off = [], 0
    for shape in shapes:
        n = math.prod(shape)
        out.append(flat[off:off + n].reshape(shape))
        off += n
    return out


def batch_pad(requests: Sequence[np.ndarray], max_rows: int = None) -> np.ndarray:
    """One layer of batch_logits_and_key_value_memory_dict (kv_cache_batch.py:
    11-22): each request's [b_i, S_i, ...] is zero-padded at the end of dim 1
    to max_rows (default max S_i) and the requests are stacked along dim 0."""
    if max_rows is None:
        max_rows = max(r.shape[1] for r in requests)
    parts = []
    for r in requests:
        if r.shape[1] > max_rows:
            raise ValueError("request longer than max_rows")
        padded = np.zeros((r.shape[0], max_rows) + r.shape[2:], dtype=r.dtype)
        padded[:, :r.shape[1]] = r
        parts.append(padded)
    return np.concatenate(parts, axis=0)


def concat_dim(shards: Sequence[np.ndarray], dim: int = 3) -> np.ndarray:
    """One key of concat_dicts: the tensor-parallel shards concatenated along
    `dim`, the KV-head dimension of [B, S, 2, H, D] by default
    (tensor_parallel_dim_concat.py:9-19)."""
    return np.concatenate(list(shards), axis=dim)


# ------------------------------------------------------ FasterTransformer ---


def ft_layout(cache: np.ndarray, pack: int):
    """[B, S, 2, H, D] -> (K [B, H, D/pack, S, pack], V [B, H, S, D]): the
    rearranges 'b s h (d packsize) -> b h d s packsize' and
    'b s h d -> b h s d' of mha.py:296-298."""
    b, s, _, h, d = cache.shape
    k = cache[:, :, 0].reshape(b, s, h, d // pack, pack).transpose(0, 2, 3, 1, 4)
    v = cache[:, :, 1].transpose(0, 2, 1, 3)
    return np.ascontiguousarray(k), np.ascontiguousarray(v)


def ft_unlayout(k: np.ndarray, v: np.ndarray) -> np.ndarray:
    """Inverse of ``ft_layout``: the FT pair back to [B, S, 2, H, D]."""
    b, h, dp, s, p = k.shape
    kk = k.transpose(0, 3, 1, 2, 4).reshape(b, s, h, dp * p)
    vv = v.transpose(0, 2, 1, 3)
    return np.stack([kk, vv], axis=2)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """x rounded to ``dtype`` ("float16", "bfloat16", "float32"), nearest
    even, returned as float64."""
    x32 = np.asarray(x, dtype=np.float64).astype(np.float32)
    if dtype == "float32":
        return x32.astype(np.float64)
    if dtype == "float16":
        return x32.astype(np.float16).astype(np.float64)
    if dtype == "bfloat16":
        bits = x32.view(np.uint32).astype(np.uint64)
        bits = (bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000
        return bits.astype(np.uint32).view(np.float32).astype(np.float64)
    raise ValueError(dtype)


def rotary(x: np.ndarray, pos: int, rot_dim: int, base: float, neox: bool) -> np.ndarray:
    """Rotary embedding of x [..., D] at position ``pos`` (float64): pair j of
    the first rot_dim dimensions -- (j, j + rot_dim/2) in the GPT-NeoX form,
    (2j, 2j + 1) in the GPT-J form -- turns by pos * base^(-2j / rot_dim)."""
    out = np.array(x, dtype=np.float64)
    half = rot_dim // 2
    for j in range(half):
        theta = pos * base ** (-2.0 * j / rot_dim)
        c, s = math.cos(theta), math.sin(theta)
        i0, i1 = (j, j + half) if neox else (2 * j, 2 * j + 1)
        x0, x1 = out[..., i0].copy(), out[..., i1].copy()
        out[..., i0] = x0 * c - x1 * s
        out[..., i1] = x0 * s + x1 * c
    return out


def ft_decode(q, k_new, v_new, k_ft, v_ft, positions, rot_dim=0, base=10000.0, neox=True,
              dtype="float32", softmax_scale=None):
    """One FT decode step (mha.py:310-337): q [B, Hq, D], k_new/v_new
    [B, Hkv, D], FT caches; sequence b's token sits at positions[b].  q and
    k are rotated there and rounded to ``dtype``; k and v are written at that
    position; q attends to [0, position].  Returns (out [B, Hq, D] float64,
    K', V') with the caches' dtype preserved."""
    pack = k_ft.shape[-1]
    cache = ft_unlayout(np.asarray(k_ft), np.asarray(v_ft)).astype(np.float64)
    batch = q.shape[0]
    qr = np.stack([round_to(rotary(q[b], positions[b], rot_dim, base, neox), dtype) for b in range(batch)])
    kr = np.stack([round_to(rotary(k_new[b], positions[b], rot_dim, base, neox), dtype)
                   for b in range(batch)])
    for b in range(batch):
        cache[b, positions[b], 0] = kr[b]
        cache[b, positions[b], 1] = np.asarray(v_new[b], dtype=np.float64)
    out = attend(qr[:, None], cache, [p + 1 for p in positions], softmax_scale=softmax_scale)[:, 0]
    k2, v2 = ft_layout(cache, pack)
    return out, k2.astype(np.asarray(k_ft).dtype), v2.astype(np.asarray(v_ft).dtype)
