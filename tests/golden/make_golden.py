"""Writes the golden fixtures under tests/golden/ (run once, on the CPU).

* ``fixture_seed17/`` -- the reference's synthetic correctness checkpoint,
  rebuilt by its recipe (hexgen2/fixture.py:13-17: torch.manual_seed(17),
  LlamaConfig(vocab 128, hidden 128, intermediate 256, 2 layers, 4 heads,
  2 KV heads, 128 positions), HuggingFace random init).  The reference's
  native fp16 GPU engine recorded its greedy tokens for the validator's
  prompts (hexgen2/validate.py:22-23): [120], [120, 120, 120, 120],
  [117, 30, 58] (evidence/2026-10-19/fabric-pilot.json:743-786).
* ``tiny_llama/`` -- the 2-layer, hidden-64, 4-head, head-dim-16,
  vocab-256 decoder with seeded N(0, 0.02) weights, and its 16-token prompt.
* ``greedy.json`` -- greedy tokens of both models by full-context recompute
  without a cache (the validator's reference semantics, hexgen2/validate.py:
  26-33) with HuggingFace ``LlamaForCausalLM`` eager in float32 on the CPU,
  plus the top-2 logit margin of every step so near-ties are visible.
* ``packet_bytes.json`` -- KV packet sizes the reference recorded
  (``kv_packet_bytes``) with the model geometry that produced them.

HuggingFace transformers is used as an independent implementation of the
Llama architecture, never the reference's code.
"""
from __future__ import annotations

import json
from pathlib import Path

import torch
from transformers import LlamaConfig, LlamaForCausalLM

HERE = Path(__file__).resolve().parent

TINY_SEED = 20260101
TINY_PROMPT_SEED = 7


def _greedy(model, prompt, count):
    ids = torch.tensor([prompt], dtype=torch.long)
    tokens, margins = [], []
    with torch.inference_mode():
        for _ in range(count):
            logits = model(ids).logits[:, -1].float()
            top = logits.topk(2)
            token = int(top.indices[0, 0])
            tokens.append(token)
            margins.append(float(top.values[0, 0] - top.values[0, 1]))
            ids = torch.cat((ids, torch.tensor([[token]])), dim=1)
    return tokens, margins


def _save(model, folder: Path, note: dict):
    folder.mkdir(parents=True, exist_ok=True)
    model.save_pretrained(folder, safe_serialization=True)
    (folder / "fixture.json").write_text(json.dumps(note, indent=2) + "\n")


def main():
    greedy = {}

    torch.manual_seed(17)
    config = LlamaConfig(vocab_size=128, hidden_size=128, intermediate_size=256,
                         num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                         max_position_embeddings=128, bos_token_id=1, eos_token_id=2, pad_token_id=0)
    model = LlamaForCausalLM(config).eval()
    _save(model, HERE / "fixture_seed17", {"kind": "synthetic-random-weights", "seed": 17,
                                            "recipe": "hexgen2/fixture.py:13-17"})
    cases = []
    recorded = {(1, 1): [120], (4, 4): [120, 120, 120, 120], (7, 3): [117, 30, 58]}
    for (length, count), evidence in recorded.items():
        prompt = list(range(1, length + 1))
        tokens, margins = _greedy(model, prompt, count)
        cases.append({"prompt": prompt, "max_new_tokens": count, "hf_fp32_tokens": tokens,
                      "top2_margins": margins, "reference_gpu_fp16_tokens": evidence,
                      "evidence": "evidence/2026-10-19/fabric-pilot.json:743-786"})
    greedy["fixture_seed17"] = cases

    torch.manual_seed(TINY_SEED)
    config = LlamaConfig(vocab_size=256, hidden_size=64, intermediate_size=128,
                         num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=4,
                         max_position_embeddings=64, initializer_range=0.02,
                         bos_token_id=1, eos_token_id=2, pad_token_id=0)
    model = LlamaForCausalLM(config).eval()
    _save(model, HERE / "tiny_llama", {"kind": "synthetic-random-weights", "seed": TINY_SEED,
                                        "init": "N(0, 0.02)"})
    generator = torch.Generator().manual_seed(TINY_PROMPT_SEED)
    prompt = torch.randint(0, 256, (16,), generator=generator).tolist()
    tokens, margins = _greedy(model, prompt, 8)
    greedy["tiny_llama"] = [{"prompt": prompt, "max_new_tokens": 8, "hf_fp32_tokens": tokens,
                             "top2_margins": margins}]
    (HERE / "greedy.json").write_text(json.dumps(greedy, indent=2) + "\n")

    # kv_packet_bytes recorded by the reference pilot, with the geometry of
    # the model that produced them (2 layers x 2 KV heads x 32 dims fp16 for
    # the fixture; TinyLlama-1.1B: 22 layers x 4 KV heads x 64 dims fp16).
    packets = {
        "source": "evidence/2026-10-19/fabric-pilot.json",
        "cases": [
            {"line": 81, "model": "fixture", "layers": 2, "kv_heads": 2, "head_dim": 32, "elem_bytes": 2, "prompt_tokens": 1, "kv_packet_bytes": 520},
            {"line": 98, "model": "fixture", "layers": 2, "kv_heads": 2, "head_dim": 32, "elem_bytes": 2, "prompt_tokens": 4, "kv_packet_bytes": 2056},
            {"line": 114, "model": "fixture", "layers": 2, "kv_heads": 2, "head_dim": 32, "elem_bytes": 2, "prompt_tokens": 7, "kv_packet_bytes": 3592},
            {"line": 198, "model": "tinyllama", "layers": 22, "kv_heads": 4, "head_dim": 64, "elem_bytes": 2, "prompt_tokens": 13, "kv_packet_bytes": 292872},
            {"line": 227, "model": "tinyllama", "layers": 22, "kv_heads": 4, "head_dim": 64, "elem_bytes": 2, "prompt_tokens": 14, "kv_packet_bytes": 315400},
            {"line": 309, "model": "tinyllama", "layers": 22, "kv_heads": 4, "head_dim": 64, "elem_bytes": 2, "prompt_tokens": 82, "kv_packet_bytes": 1847304},
            {"line": 323, "model": "tinyllama", "layers": 22, "kv_heads": 4, "head_dim": 64, "elem_bytes": 2, "prompt_tokens": 6, "kv_packet_bytes": 135176},
        ],
    }
    (HERE / "packet_bytes.json").write_text(json.dumps(packets, indent=2) + "\n")


if __name__ == "__main__":
    main()
