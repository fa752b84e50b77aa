"""Writes tests/golden/trace_tokens.json: greedy tokens of the requests in
tests/golden/tiny-trace.jsonl (the reference pilot's trace,
configs/tiny-trace.jsonl) on the seed-17 fixture checkpoint, by full-context
recompute without a cache (hexgen2/validate.py:26-33 semantics) with
HuggingFace ``LlamaForCausalLM`` eager in float32 on the CPU, plus the top-2
logit margin of every step.  HuggingFace is an independent implementation of
the architecture, never the reference's code."""
from __future__ import annotations

import json
from pathlib import Path

import torch
from transformers import LlamaForCausalLM

HERE = Path(__file__).resolve().parent


def main():
    model = LlamaForCausalLM.from_pretrained(HERE / "fixture_seed17", local_files_only=True,
                                             torch_dtype=torch.float32, attn_implementation="eager").eval()
    out = {}
    for line in (HERE / "tiny-trace.jsonl").read_text().splitlines():
        row = json.loads(line)
        ids = torch.tensor([row["input_ids"]], dtype=torch.long)
        tokens, margins = [], []
        with torch.inference_mode():
            for _ in range(row["max_new_tokens"]):
                logits = model(ids).logits[:, -1].float()
                top = logits.topk(2)
                tokens.append(int(top.indices[0, 0]))
                margins.append(float(top.values[0, 0] - top.values[0, 1]))
                ids = torch.cat((ids, top.indices[:, :1]), dim=1)
        out[row["id"]] = {"hf_fp32_tokens": tokens, "top2_margins": margins}
    (HERE / "trace_tokens.json").write_text(json.dumps(out, indent=2) + "\n")


if __name__ == "__main__":
    main()
