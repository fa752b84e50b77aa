"""Writes tests/golden/hf_logits.json: HuggingFace full-context logits for
every prompt the engine tests decode, so the tests can apply the reference
validator's logit check (hexgen2/validate.py:33-43:
``torch.allclose(logits, reference_logits, atol=0.03, rtol=0.03)`` against
``LlamaForCausalLM`` eager in the engine's own dtype) at prefill and at
every decode step.

For each committed checkpoint (``fixture_seed17``, ``tiny_llama``) and each
prompt -- the validator's prompts ``range(1, L + 1)`` for (L, n) in
{(1, 1), (4, 4), (7, 3)} and the pilot trace's requests on the fixture, the
16-token prompt on the tiny Llama -- the model runs eager on the CPU in
float32, float16 and bfloat16 over the prompt followed by the float32 greedy
tokens recorded in greedy.json / trace_tokens.json (so every dtype is read
along one token path).  Step i's logits are those of the last position of
prompt + tokens[:i], without a KV cache (validate.py:26-33 semantics).
HuggingFace is an independent implementation of the architecture, never the
reference's code.  Run once on the CPU: ``python tests/golden/make_logits.py``.
"""
from __future__ import annotations

import json
from pathlib import Path

import torch
from transformers import LlamaForCausalLM

HERE = Path(__file__).resolve().parent
DTYPES = ("float32", "float16", "bfloat16")


def step_logits(model, prompt, tokens, dtype):
    out = []
    ids = list(prompt)
    with torch.inference_mode():
        for i in range(len(tokens)):
            logits = model(torch.tensor([ids], dtype=torch.long)).logits[0, -1].float()
            out.append([round(float(x), 6) for x in logits])
            ids.append(tokens[i])
    return out


def main():
    torch.set_num_threads(8)
    greedy = json.loads((HERE / "greedy.json").read_text())
    trace = json.loads((HERE / "trace_tokens.json").read_text())
    requests = [json.loads(s) for s in (HERE / "tiny-trace.jsonl").read_text().splitlines() if s.strip()]
    cases = {
        "fixture_seed17": [(c["prompt"], c["hf_fp32_tokens"]) for c in greedy["fixture_seed17"]]
        + [(r["input_ids"], trace[r["id"]]["hf_fp32_tokens"]) for r in requests],
        "tiny_llama": [(c["prompt"], c["hf_fp32_tokens"]) for c in greedy["tiny_llama"]],
    }
    out = {"note": "HuggingFace LlamaForCausalLM eager on CPU; logits[i] = last-position logits of "
                   "prompt + hf_fp32_tokens[:i] (no KV cache)", "models": {}}
    for name, items in cases.items():
        per_model = []
        models = {d: LlamaForCausalLM.from_pretrained(HERE / name, local_files_only=True, torch_dtype=getattr(torch, d),
                                                      attn_implementation="eager").eval() for d in DTYPES}
        for prompt, tokens in items:
            per_model.append({"prompt": prompt, "hf_fp32_tokens": tokens,
                              "logits": {d: step_logits(models[d], prompt, tokens, d) for d in DTYPES}})
        out["models"][name] = per_model
    (HERE / "hf_logits.json").write_text(json.dumps(out) + "\n")


if __name__ == "__main__":
    main()
