"""Prefill/decode engine with the KV handoff on the GPU.

Mirrors the pilot's ``Engine`` (hexgen2/model.py:22-124): same constructor,
``prefill(input_ids, max_new_tokens) -> (first_token, cache, logits)`` and
``decode(first_token, cache, prompt_length, max_new_tokens, on_token=None)``,
same cache dict contract ``{layer: [1, L, 2, kv_heads, head_dim]}`` and the
same validation errors.  What changes is where the bytes go:

* prefill ends with ONE hexkv pack launch that gathers the live rows of every
  layer into one contiguous handoff buffer; the returned dict holds
  per-layer views of that buffer (model.py:81 did one copy per layer);
* decode starts with ONE hexkv unpack launch that scatters the received
  layers into a single preallocated decode cache (model.py:104-108 allocated
  and copied per layer);
* each decode step appends and attends through hexkv (mha.py:286, 568-569).
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import torch

from . import ops
from .generation import CacheState
from .llama import LlamaHost, LlamaShape, read_config
from .mha import check_kv_status


# Packed handoff buffers at or above this size are allocated per layer, so
# that each stays an allocation another process can map (below 2 GiB).
PER_LAYER_HANDOFF_BYTES = 1 << 30


def model_identity(model_dir) -> dict:
    """SHA-256 of every checkpoint/config file and of their listing, as the
    pilot records it (hexgen2/record.py:36-45)."""
    files = sorted(p for p in Path(model_dir).iterdir() if p.is_file() and (
        p.suffix in {".safetensors", ".json"} or p.name == "tokenizer.model"))
    hashes = {p.name: hashlib.sha256(p.read_bytes()).hexdigest() for p in files}
    if not any(name.endswith(".safetensors") for name in hashes):
        raise ValueError("No safetensors checkpoint in model directory")
    return {"files": hashes, "sha256": hashlib.sha256(json.dumps(hashes, sort_keys=True).encode()).hexdigest()}


class Engine:
    def __init__(self, model_dir, engine="native", device="cuda", dtype="float16",
                 fused_append: bool = False):
        self.device, self.dtype = torch.device(device), getattr(torch, dtype)
        self.shape = LlamaShape.from_config(read_config(model_dir))
        self.identity = model_identity(model_dir)
        self.kind = engine
        if engine != "native":
            raise ValueError("Only the native engine runs on the hexkv data path; the "
                             "hf-reference engine is the reference's CPU validator")
        if self.device.type != "cuda" or not torch.cuda.is_available():
            raise ValueError("The hexkv engine requires a HIP GPU (torch.cuda on ROCm)")
        self.model = LlamaHost.load(model_dir, self.device, self.dtype)
        self.fused_append = fused_append
        self.config = self.shape

    def _cache_geometry(self):
        s = self.shape
        return s.num_hidden_layers, s.num_key_value_heads, s.head_dim

    @torch.inference_mode()
    def prefill(self, input_ids, max_new_tokens):
        ids = torch.tensor([input_ids], dtype=torch.long, device=self.device)
        state = CacheState(len(input_ids) + max_new_tokens)
        logits = self.model.forward(ids, inference_params=state, last_token_only=True)
        n_layers = len(state.key_value_memory_dict)
        layers = [state.key_value_memory_dict[i] for i in range(n_layers)]
        # Send only initialized prompt positions, never the unused capacity:
        # one launch gathers every layer into one handoff buffer (per-layer
        # buffers when it would be too large to map from another process).
        row_shape = layers[0].shape[2:]
        nbytes = n_layers * len(input_ids) * layers[0][0, 0].numel() * layers[0].element_size()
        if nbytes >= PER_LAYER_HANDOFF_BYTES:
            out = [torch.empty((len(input_ids), *row_shape), dtype=self.dtype, device=self.device)
                   for _ in range(n_layers)]
            packed = ops.pack_live(layers, [len(input_ids)], out=out)
        else:
            packed = ops.pack_live(layers, [len(input_ids)])
        cache = {i: packed[i].unsqueeze(0) for i in range(n_layers)}
        return logits.argmax(-1), cache, logits

    @torch.inference_mode()
    def decode(self, first_token, cache, prompt_length, max_new_tokens, on_token=None, *, on_logits=None):
        """Greedy decode from the handed-off cache (model.py:86-120).
        ``on_logits`` (an addition) receives each decode step's logits
        ``[1, vocab]``, for logit-level checks."""
        token = first_token.to(self.device).reshape(1)
        generated = [int(token.item())]
        if on_token:
            on_token(generated[-1])
        n_layers, kv_heads, head_dim = self._cache_geometry()
        if set(cache) != set(range(n_layers)):
            raise ValueError("KV cache does not match the configured layer count")
        expected = (1, prompt_length, 2, kv_heads, head_dim)
        for value in cache.values():
            if tuple(value.shape) != expected or value.dtype != self.dtype:
                raise ValueError("KV cache shape/dtype does not match checkpoint and prompt")
        state = CacheState(prompt_length + max_new_tokens)
        state.sequence_len_offset = prompt_length
        # One decode cache for all layers; rows >= prompt_length stay
        # uninitialised as in model.py:105.
        full = torch.empty((n_layers, 1, state.max_sequence_len, 2, kv_heads, head_dim),
                           device=self.device, dtype=self.dtype)
        live = [cache[i].to(self.device) for i in range(n_layers)]
        live = [t if t.is_contiguous() else t.contiguous() for t in live]
        ops.unpack_live(live, full, [prompt_length])
        for i in range(n_layers):
            state.key_value_memory_dict[i] = full[i]
        ops.device_status(self.device)  # report only what this decode's kernels meet
        for _ in range(max_new_tokens - 1):
            logits = self.model.forward(token[:, None], inference_params=state, last_token_only=True,
                                        fused_append=self.fused_append)
            state.sequence_len_offset += 1
            if on_logits:
                on_logits(logits)
            token = logits.argmax(-1)
            generated.append(int(token.item()))
            # the token read synchronised: report any out-of-contract device
            # position the step's kernels met (mha.py:281-282's assert)
            check_kv_status(self.device)
            if on_token:
                on_token(generated[-1])
        return generated

    def synchronize(self):
        if self.device.type == "cuda":
            torch.cuda.synchronize(self.device)
