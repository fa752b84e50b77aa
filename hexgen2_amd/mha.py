"""Drop-in replacements for the KV-cache calls of hexgen_core's attention module.

* ``_update_kv_cache(kv, inference_params, layer_idx)`` -- append (and the
  prefill write) into the per-layer cache; hexgen/hexgen_core/modules/
  mha.py:255-288.
* ``inference_cache(...)`` -- one layer's cache in the shapes of
  ``MHA.allocate_inference_cache`` (mha.py:414-428): the ``[B, S, 2, H, D]``
  cache, or with ``fused_ft_kernel=True`` the FasterTransformer (FT) K/V pair.
* ``check_kv_status()`` -- the device-side capacity check of ragged appends
  (mha.py:281-282), reported at the caller's next synchronisation.
* ``_apply_rotary_single_query_attention(...)`` -- the FT decode step
  (mha.py:310-337): rotary, append and attention over the FT caches.
* ``FlashCrossAttention`` -- the attention module the reference's MHA calls at
  decode (mha.py:105-142); same constructor and ``forward`` signature.

Every data movement and every attention runs as a hexkv HIP kernel; CPU
tensors are rejected.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import nn

from . import ops


def inference_cache(batch_size: int, max_seqlen: int, num_heads_kv: int, head_dim: int,
                    dtype: torch.dtype, device, fused_ft_kernel: bool = False):
    """One layer's cache in the shapes ``MHA.allocate_inference_cache``
    gives it: ``torch.empty(batch, max_seqlen, 2, kv_heads, head_dim)``
    (mha.py:418-420), or with ``fused_ft_kernel`` the FT pair ``(K [batch,
    kv_heads, head_dim / pack, max_seqlen, pack], V [batch, kv_heads,
    max_seqlen, head_dim])``, pack = 4 for float32 and 8 for 16-bit data
    (mha.py:421-428).  The head geometry, dtype and device are arguments here
    (the reference method reads them from the module); the reference method
    itself needs no replacement, since it only calls ``torch.empty``."""
    if not fused_ft_kernel:
        return torch.empty(batch_size, max_seqlen, 2, num_heads_kv, head_dim, dtype=dtype, device=device)
    assert dtype in (torch.float16, torch.bfloat16, torch.float32)
    k_shape, v_shape = ops.ft_cache_shapes(batch_size, num_heads_kv, max_seqlen, head_dim, dtype)
    return (torch.empty(k_shape, dtype=dtype, device=device), torch.empty(v_shape, dtype=dtype, device=device))


# Attribute of the cache view _update_kv_cache returns for a ragged decode
# step: (seqlens, bias) with sequence b attending seqlens[b] + bias keys.
_SEQLENS_ATTR = "_hexkv_seqlens"


def _sample_positions(inference_params, batch_start: int, batch_end: int) -> Optional[torch.Tensor]:
    """``lengths_per_sample[batch_start:batch_end]`` as a contiguous int32
    device tensor (each sequence's cached length, i.e. the position its next
    token is written at), or None when the batch shares
    ``sequence_len_offset``.  ``lengths_per_sample`` is the field the
    reference reads per-sample positions from (generation.py:30, used at
    mha.py:327-328), and only for decode steps: at ``sequence_len_offset``
    0 (the prompt, where the reference's generation loop has already set it
    to the prompt lengths, generation.py:380) the write goes to the offset."""
    lengths = inference_params.lengths_per_sample
    if lengths is None or inference_params.sequence_len_offset == 0:
        return None
    if lengths.dim() != 1 or lengths.shape[0] < batch_end:
        raise ValueError(f"lengths_per_sample of shape {tuple(lengths.shape)} does not cover "
                         f"sequences [{batch_start}, {batch_end})")
    positions = lengths[batch_start:batch_end]
    if positions.dtype != torch.int32 or not positions.is_contiguous():
        positions = positions.to(torch.int32).contiguous()
    return positions


def _update_kv_cache(kv: torch.Tensor, inference_params, layer_idx: int) -> torch.Tensor:
    """kv: (batch, seqlen, 2, kv_heads, head_dim).  Writes kv at
    ``[batch_size_offset:+batch, sequence_len_offset:+seqlen]`` of layer
    ``layer_idx``'s cache (allocated on first use) and returns the view
    ``cache[batch_start:batch_end, :sequence_end]`` (mha.py:255-288).

    Ragged decode: when ``inference_params.lengths_per_sample`` is set and
    seqlen is 1, sequence b's row is written at ``lengths_per_sample[b]``
    instead (the reference keeps one offset for the whole batch,
    mha.py:276-279, and reads per-sample positions only on the FT path,
    mha.py:327-328).  ``sequence_len_offset`` must then bound every sample's
    position (the returned view spans ``sequence_len_offset + 1`` positions),
    and the view carries the per-sample key counts so that
    ``FlashCrossAttention`` attends ``lengths_per_sample[b] + 1`` keys of
    row b rather than the whole view.  The positions live in device memory,
    so the reference's capacity assert (mha.py:281-282) becomes a device
    check: a position past the cache is not written, a row past the view is
    cut to it, and ``check_kv_status`` raises ValueError for either at the
    caller's next synchronisation."""
    if inference_params.fused_ft_kernel:
        return _update_ft_cache(kv, inference_params, layer_idx)
    num_heads, head_dim = kv.shape[-2:]
    cache = inference_params.key_value_memory_dict.get(layer_idx)
    if cache is None:
        cache = inference_cache(inference_params.max_batch_size, inference_params.max_sequence_len,
                                num_heads, head_dim, kv.dtype, kv.device)
        inference_params.key_value_memory_dict[layer_idx] = cache
    batch_start = inference_params.batch_size_offset
    batch_end = batch_start + kv.shape[0]
    sequence_start = inference_params.sequence_len_offset
    sequence_end = sequence_start + kv.shape[1]
    assert batch_end <= cache.shape[0]
    assert sequence_end <= cache.shape[1]
    kv = kv.contiguous()
    target = cache[batch_start:batch_end]
    positions = _sample_positions(inference_params, batch_start, batch_end) if kv.shape[1] == 1 else None
    if positions is not None:
        ops.append_kv(target, kv.reshape(kv.shape[0], -1), positions)
    elif kv.shape[1] == 1:
        ops.append_kv(target, kv.reshape(kv.shape[0], -1), position_bias=sequence_start)
    elif kv.shape[1] > 1:
        # A multi-position write (prefill) is an unpack of one packed layer with
        # uniform lengths into the cache shifted by sequence_start rows.
        ops.unpack_live([kv.reshape(-1)], [target[:, sequence_start:]], [kv.shape[1]] * kv.shape[0])
    view = cache[batch_start:batch_end, :sequence_end]
    if positions is not None:
        setattr(view, _SEQLENS_ATTR, (positions, 1))
    return view


def _update_ft_cache(kv: torch.Tensor, inference_params, layer_idx: int) -> torch.Tensor:
    """The FT branch of _update_kv_cache (mha.py:289-305), prefill only
    (``sequence_len_offset == 0``): kv's positions ``[0, seqlen)`` go into the
    layer's FT caches, allocated on first use.  (The reference first fills a
    ``[B, S, 2, H, D]`` cache and converts all of it, mha.py:295-299; the
    positions it writes are the same, the rest is uninitialised either way.)
    Returns ``kv`` as the reference does."""
    assert inference_params.sequence_len_offset == 0
    assert kv.dtype in (torch.float16, torch.bfloat16, torch.float32)
    num_heads, head_dim = kv.shape[-2:]
    caches = inference_params.key_value_memory_dict.get(layer_idx)
    if caches is None:
        caches = inference_cache(inference_params.max_batch_size, inference_params.max_sequence_len,
                                 num_heads, head_dim, kv.dtype, kv.device, fused_ft_kernel=True)
        inference_params.key_value_memory_dict[layer_idx] = caches
    k_cache, v_cache = caches
    batch_start = inference_params.batch_size_offset
    batch_end = batch_start + kv.shape[0]
    assert batch_end <= v_cache.shape[0]
    assert kv.shape[1] <= v_cache.shape[2]
    ops.ft_store(kv, k_cache[batch_start:batch_end], v_cache[batch_start:batch_end])
    return kv


def _apply_rotary_single_query_attention(qkv: torch.Tensor, inference_params, layer_idx: int,
                                         rotary_emb_dim: int, rotary_emb_base: float, kv=None,
                                         rotary_emb_interleaved: bool = False) -> torch.Tensor:
    """One FT decode step of layer ``layer_idx`` (mha.py:310-337).

    qkv ``(B, 1, 3, H, D)`` when kv is None, else q ``(B, 1, H, D)`` with kv
    ``(B, 1, 2, H_k, D)``.  The new token sits at ``lengths_per_sample[b]``
    when the inference params carry per-sample lengths, else at
    ``sequence_len_offset``; q and k are rotated there (``rotary_emb_dim``
    leading dimensions, GPT-NeoX halves unless ``rotary_emb_interleaved``), k
    and v are written to the FT caches and q attends to positions
    ``[0, position]``.  Returns ``(B, 1, H, D)``."""
    assert inference_params.fused_ft_kernel
    if kv is None:
        q, k, v = qkv[:, 0].unbind(dim=1)
    else:
        q = qkv[:, 0]
        k, v = kv[:, 0].unbind(dim=1)
    batch_start = inference_params.batch_size_offset
    batch_end = batch_start + q.shape[0]
    k_cache, v_cache = inference_params.key_value_memory_dict[layer_idx]
    lengths = inference_params.lengths_per_sample
    if lengths is not None:
        positions = lengths[batch_start:batch_end].to(torch.int32).contiguous()
        bias, max_position = 0, v_cache.shape[2] - 1
    else:
        positions, bias = None, inference_params.sequence_len_offset
        max_position = bias
    if k.stride() != v.stride():
        k, v = k.contiguous(), v.contiguous()
    context = ops.ft_attend(q, k, v, k_cache[batch_start:batch_end], v_cache[batch_start:batch_end],
                            max_position=max_position, positions=positions, position_bias=bias,
                            rotary_dim=rotary_emb_dim, rotary_base=rotary_emb_base,
                            rotary_neox=not rotary_emb_interleaved)
    return context.unsqueeze(1)


class FlashCrossAttention(nn.Module):
    """Scaled dot-product attention of q against a packed KV tensor.

    Same interface as hexgen_core's FlashCrossAttention (mha.py:87-142):
    q (B, Sq, H, D), kv (B, Sk, 2, H_k, D) -> (B, Sq, H, D), GQA when
    H_k < H.  With ``causal`` and Sq > 1 query t sees keys < Sk - Sq + t + 1
    (the prefill triangle when Sq == Sk).  float32 is accepted too (the
    reference routes it to CrossAttention, mha.py:195-244).  Dropout is not
    applied (inference only).
    """

    def __init__(self, causal=False, softmax_scale=None, attention_dropout=0.0):
        super().__init__()
        self.causal = causal
        self.softmax_scale = softmax_scale
        self.drop = nn.Dropout(attention_dropout)

    def forward(self, q, kv, causal=None, cu_seqlens=None, max_seqlen=None,
                cu_seqlens_k=None, max_seqlen_k=None, *, seqlens_k=None):
        """``seqlens_k`` (device int32 ``[B]``, an addition to the reference
        signature) makes row b attend only its first ``seqlens_k[b]`` keys of
        the ``Sk`` in ``kv`` (a ragged decode batch in a padded cache).  A
        view returned by ``_update_kv_cache`` for a ragged step carries these
        counts itself, so the reference's call ``inner_cross_attn(q, kv,
        causal=False)`` (mha.py:568-569) needs no change."""
        assert q.dtype in (torch.float16, torch.bfloat16, torch.float32)
        assert q.is_cuda and kv.is_cuda
        if cu_seqlens is not None or cu_seqlens_k is not None:
            raise NotImplementedError("variable-length (cu_seqlens) attention is not supported")
        causal = self.causal if causal is None else causal
        batch_size = q.shape[0]
        seqlen_k = kv.shape[1]
        assert kv.shape[0] == batch_size and kv.shape[4] == q.shape[3]
        bias = seqlen_k
        if seqlens_k is None and getattr(kv, _SEQLENS_ATTR, None) is not None:
            seqlens_k, bias = getattr(kv, _SEQLENS_ATTR)
            bias = int(bias)
        elif seqlens_k is not None:
            bias = 0
        if seqlens_k is not None:
            assert seqlens_k.dtype == torch.int32 and seqlens_k.is_cuda and seqlens_k.numel() == batch_size
            seqlens_k = seqlens_k.contiguous()
        q = q if q.stride(-1) == 1 and q.stride(-2) == q.shape[-1] else q.contiguous()
        if kv.stride(-1) != 1 or kv.stride(-2) != kv.shape[-1] or kv.stride(1) != kv[0, 0].numel():
            kv = kv.contiguous()
        return ops.decode_attention(q, kv, max_seqlen=seqlen_k, seqlens=seqlens_k, seqlen_bias=bias,
                                    causal=bool(causal) and q.shape[1] > 1,
                                    softmax_scale=self.softmax_scale)


def check_kv_status(device=None) -> None:
    """Raise ValueError if a cache append or attention since the last check
    met a per-sample position (``lengths_per_sample``) outside the cache or
    the attended view: the device-side form of the reference's capacity
    assert (mha.py:281-282).  It synchronises the current stream; decode
    loops call it where they read the token anyway."""
    ops.check_device_status(device)


def update_and_attend(q: torch.Tensor, kv: torch.Tensor, inference_params, layer_idx: int,
                      softmax_scale: Optional[float] = None) -> torch.Tensor:
    """The decode-step pair ``_update_kv_cache`` + ``inner_cross_attn(q, kv,
    causal=False)`` (mha.py:565-569) as one fused HIP launch: the new row is
    written to the cache and attended from registers.  q (B, 1, H, D),
    kv (B, 1, 2, H_k, D).  With ``lengths_per_sample`` set, row b is written
    at ``lengths_per_sample[b]`` and attends that many keys plus the new one;
    ``sequence_len_offset`` bounds every sample's position (checked on the
    device, reported by ``check_kv_status``)."""
    cache = inference_params.key_value_memory_dict[layer_idx]
    batch_start = inference_params.batch_size_offset
    batch_end = batch_start + kv.shape[0]
    offset = inference_params.sequence_len_offset
    assert kv.shape[1] == 1 and q.shape[1] == 1
    assert batch_end <= cache.shape[0] and offset + 1 <= cache.shape[1]
    target = cache[batch_start:batch_end]
    positions = _sample_positions(inference_params, batch_start, batch_end)
    return ops.decode_attention(q.contiguous(), target, max_seqlen=offset + 1, seqlens=positions,
                                seqlen_bias=0 if positions is not None else offset,
                                kv_new=kv.contiguous(), softmax_scale=softmax_scale)
