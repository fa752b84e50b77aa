"""Minimal Llama decoder host that drives the KV data path through its real call sites.

It plays the role of hexgen_core's GPTLMHeadModel for the Llama subset the
pilot runs (pre-norm blocks, RMSNorm, rotary q/k, GQA attention with a KV
cache, SwiGLU MLP, untied LM head; hexgen/hexgen_core/models/gpt.py:363-483,
modules/block.py:112-175, mlp.py:63-87, rms_norm.py:6-15).  Weights are read
in HuggingFace Llama layout from safetensors.  Per layer and step the cache
calls are exactly the reference's: ``_update_kv_cache`` then
``FlashCrossAttention`` (mha.py:565-569), or the fused HIP append+attend;
with ``fused_ft_kernel`` the decode steps call
``_apply_rotary_single_query_attention`` on unrotated q/k (mha.py:553-571).
Dense projections use torch (hipBLASLt); every KV byte moves through hexkv.
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path

import torch
import torch.nn.functional as F

from .mha import FlashCrossAttention, _apply_rotary_single_query_attention, _update_kv_cache, update_and_attend


@dataclass
class LlamaShape:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    rms_norm_eps: float = 1e-6
    rope_theta: float = 10000.0
    max_position_embeddings: int = 2048
    tie_word_embeddings: bool = False

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    @classmethod
    def from_config(cls, config: dict) -> "LlamaShape":
        if config.get("model_type") != "llama" or config.get("rope_scaling") is not None:
            raise ValueError("This baseline supports Llama architecture without RoPE scaling")
        theta = config.get("rope_theta")
        if theta is None:
            theta = (config.get("rope_parameters") or {}).get("rope_theta", 10000.0)
        return cls(vocab_size=config["vocab_size"], hidden_size=config["hidden_size"],
                   intermediate_size=config["intermediate_size"],
                   num_hidden_layers=config["num_hidden_layers"],
                   num_attention_heads=config["num_attention_heads"],
                   num_key_value_heads=config.get("num_key_value_heads") or config["num_attention_heads"],
                   rms_norm_eps=config.get("rms_norm_eps", 1e-6), rope_theta=float(theta),
                   max_position_embeddings=config.get("max_position_embeddings", 2048),
                   tie_word_embeddings=bool(config.get("tie_word_embeddings", False)))


def read_config(model_dir) -> dict:
    return json.loads((Path(model_dir) / "config.json").read_text())


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """rms_norm.py:13-15: normalise in fp32, cast back, scale."""
    normalized = x.float() * torch.rsqrt(x.float().square().mean(-1, keepdim=True) + eps)
    return normalized.to(x.dtype) * weight


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


class LlamaHost:
    """Greedy-decode host; ``forward`` mirrors GPTLMHeadModel.forward's
    ``(input_ids, inference_params, last_token_only)`` contract."""

    def __init__(self, shape: LlamaShape, weights: dict, device, dtype):
        self.shape = shape
        self.device, self.dtype = torch.device(device), dtype
        w = {k: v.to(device=self.device, dtype=dtype) for k, v in weights.items()}
        self.embed = w["model.embed_tokens.weight"]
        self.norm = w["model.norm.weight"]
        self.lm_head = w["model.embed_tokens.weight"] if shape.tie_word_embeddings else w["lm_head.weight"]
        self.layers = []
        for i in range(shape.num_hidden_layers):
            p = f"model.layers.{i}."
            self.layers.append({
                "ln1": w[p + "input_layernorm.weight"], "ln2": w[p + "post_attention_layernorm.weight"],
                "wq": w[p + "self_attn.q_proj.weight"], "wk": w[p + "self_attn.k_proj.weight"],
                "wv": w[p + "self_attn.v_proj.weight"], "wo": w[p + "self_attn.o_proj.weight"],
                "gate": w[p + "mlp.gate_proj.weight"], "up": w[p + "mlp.up_proj.weight"],
                "down": w[p + "mlp.down_proj.weight"],
            })
        d = shape.head_dim
        self.inv_freq = 1.0 / (shape.rope_theta ** (torch.arange(0, d, 2, device=self.device,
                                                                  dtype=torch.float32) / d))
        self.scale = d ** -0.5  # gpt.py:72
        self.attn = FlashCrossAttention(causal=True, softmax_scale=self.scale)

    @classmethod
    def load(cls, model_dir, device, dtype) -> "LlamaHost":
        from safetensors.torch import load_file
        shape = LlamaShape.from_config(read_config(model_dir))
        shards = sorted(Path(model_dir).glob("*.safetensors"))
        if not shards:
            raise ValueError("A local safetensors checkpoint is required")
        state = {}
        for shard in shards:
            values = load_file(str(shard), device="cpu")
            if set(state).intersection(values):
                raise ValueError("Duplicate checkpoint keys")
            state.update(values)
        return cls(shape, state, device, dtype)

    def _rope(self, x: torch.Tensor, offset: int, positions=None) -> torch.Tensor:
        """Rotary (GPT-NeoX halves) of ``x [B, S, H, D]`` at positions
        ``offset + s``, or for one new token per sequence (S == 1) at each
        sequence's own ``positions[b]`` (a ragged decode batch)."""
        seqlen = x.shape[1]
        if positions is not None:
            freqs = positions.to(torch.float32)[:, None] * self.inv_freq[None, :]  # [B, D/2]
            emb = torch.cat((freqs, freqs), dim=-1)
            cos = emb.cos().to(x.dtype)[:, None, None, :]
            sin = emb.sin().to(x.dtype)[:, None, None, :]
            return x * cos + _rotate_half(x) * sin
        pos = torch.arange(offset, offset + seqlen, device=self.device, dtype=torch.float32)
        freqs = torch.outer(pos, self.inv_freq)
        emb = torch.cat((freqs, freqs), dim=-1)
        cos = emb.cos().to(x.dtype)[None, :, None, :]
        sin = emb.sin().to(x.dtype)[None, :, None, :]
        return x * cos + _rotate_half(x) * sin

    @torch.inference_mode()
    def forward(self, input_ids: torch.Tensor, inference_params, last_token_only: bool = True,
                fused_append: bool = False) -> torch.Tensor:
        s = self.shape
        batch, seqlen = input_ids.shape
        d = s.head_dim
        offset = inference_params.sequence_len_offset
        # A ragged decode batch: each sequence's token sits at its own cached
        # length (lengths_per_sample, generation.py:30).
        positions = None
        if inference_params.lengths_per_sample is not None and seqlen == 1 and offset > 0:
            b0 = inference_params.batch_size_offset
            positions = inference_params.lengths_per_sample[b0:b0 + batch]
        h = F.embedding(input_ids, self.embed)
        for i, layer in enumerate(self.layers):
            x = rms_norm(h, layer["ln1"], s.rms_norm_eps)
            q = (x @ layer["wq"].T).view(batch, seqlen, s.num_attention_heads, d)
            k = (x @ layer["wk"].T).view(batch, seqlen, s.num_key_value_heads, d)
            v = (x @ layer["wv"].T).view(batch, seqlen, s.num_key_value_heads, d)
            if inference_params.fused_ft_kernel and offset > 0:
                # FT decode (mha.py:553-571): rotary, append and attention in one call
                context = _apply_rotary_single_query_attention(q, inference_params, i, d, s.rope_theta,
                                                               kv=torch.stack((k, v), dim=2))
            else:
                q, k = self._rope(q, offset, positions), self._rope(k, offset, positions)
                kv = torch.stack((k, v), dim=2)  # [B, S, 2, Hkv, D]
                if fused_append and offset > 0 and seqlen == 1 and i in inference_params.key_value_memory_dict:
                    context = update_and_attend(q, kv, inference_params, i, self.scale)
                else:
                    kv_view = _update_kv_cache(kv, inference_params, i)
                    # prompt (offset 0): causal; decode: causal=False (mha.py:566-569)
                    context = self.attn(q, kv_view, causal=None if offset == 0 else False)
            h = h + context.reshape(batch, seqlen, -1) @ layer["wo"].T
            x = rms_norm(h, layer["ln2"], s.rms_norm_eps)
            h = h + (F.silu(x @ layer["gate"].T) * (x @ layer["up"].T)) @ layer["down"].T
        if last_token_only:
            h = h[:, -1]
        return rms_norm(h, self.norm, s.rms_norm_eps) @ self.lm_head.T
