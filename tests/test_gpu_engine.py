"""Greedy-token parity of the engine driving the hexkv data path end to end.

* The reference's seed-17 fixture checkpoint must decode the tokens the
  reference's native GPU engine recorded (evidence/2026-10-19/
  fabric-pilot.json:743-786) through prefill -> pack -> device handoff ->
  unpack -> append+attend decode.
* The tiny-Llama checkpoint (2 layers, hidden 64, 4 heads, head_dim 16,
  vocab 256) in fp32 must decode the golden tokens of HuggingFace
  full-context recompute.
* Transferred-cache tokens must equal the colocated run (hexgen2/run.py:
  167-176 semantics), with and without the fused append+attend.
"""
import json
from pathlib import Path

import pytest
import torch

from hexgen2_amd.engine import Engine
from hexgen2_amd.transport import DeviceChannel, recv_packet, send_packet

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
GREEDY = json.loads((GOLDEN / "greedy.json").read_text())


def run_split(engine, prompt, count):
    """Prefill, hand the cache over a same-GPU channel, decode (run.py:141-198)."""
    prefill_side, decode_side = DeviceChannel.pair()
    first, cache, _ = engine.prefill(prompt, count)
    sent = send_packet({"first": first, **{str(k): v for k, v in cache.items()}},
                       {"id": "r", "prompt_length": len(prompt)}, dst=1, channel=prefill_side)
    tensors, metadata = recv_packet(src=0, channel=decode_side)
    assert metadata == {"id": "r", "prompt_length": len(prompt)}
    tokens = engine.decode(tensors["first"], {int(k): v for k, v in tensors.items() if k != "first"},
                           len(prompt), count)
    return tokens, sent


@pytest.mark.parametrize("dtype", ["float16", "bfloat16", "float32"])
def test_fixture_tokens_match_reference_gpu_run(device, dtype):
    engine = Engine(GOLDEN / "fixture_seed17", "native", "cuda", dtype)
    for case in GREEDY["fixture_seed17"]:
        print(f"fixture {dtype} prompt={case['prompt']}", flush=True)
        tokens, sent = run_split(engine, case["prompt"], case["max_new_tokens"])
        assert tokens == case["reference_gpu_fp16_tokens"] == case["hf_fp32_tokens"]
        elem = 4 if dtype == "float32" else 2
        # int64 first token + 2 layers x L x (2 x 2 heads x 32 dims) live bytes
        assert sent == 8 + 2 * len(case["prompt"]) * 2 * 2 * 32 * elem


@pytest.mark.parametrize("fused", [False, True])
def test_tiny_llama_fp32_golden_and_colocated(device, fused):
    case = GREEDY["tiny_llama"][0]
    engine = Engine(GOLDEN / "tiny_llama", "native", "cuda", "float32", fused_append=fused)
    tokens, sent = run_split(engine, case["prompt"], case["max_new_tokens"])
    assert tokens == case["hf_fp32_tokens"]
    assert sent == 8 + 2 * 16 * (2 * 4 * 16 * 4)
    # colocated: same engine, no transfer (run.py:168-169)
    first, cache, _ = engine.prefill(case["prompt"], case["max_new_tokens"])
    assert engine.decode(first, cache, len(case["prompt"]), case["max_new_tokens"]) == tokens


def test_decode_rejects_mismatched_cache(device):
    engine = Engine(GOLDEN / "tiny_llama", "native", "cuda", "float32")
    first, cache, _ = engine.prefill([1, 2, 3], 2)
    with pytest.raises(ValueError, match="layer count"):
        engine.decode(first, {0: cache[0]}, 3, 2)
    with pytest.raises(ValueError, match="shape/dtype"):
        engine.decode(first, cache, 4, 2)
    with pytest.raises(ValueError, match="shape/dtype"):
        engine.decode(first, {k: v.half() for k, v in cache.items()}, 3, 2)


def test_prefill_cache_is_one_packed_buffer(device):
    engine = Engine(GOLDEN / "fixture_seed17", "native", "cuda", "float16")
    first, cache, logits = engine.prefill([1, 2, 3, 4, 5], 3)
    assert sorted(cache) == [0, 1]
    assert all(tuple(v.shape) == (1, 5, 2, 2, 32) and v.is_contiguous() for v in cache.values())
    # layer 1 starts right after layer 0: one contiguous handoff buffer
    assert cache[1].data_ptr() == cache[0].data_ptr() + cache[0].numel() * cache[0].element_size()
    assert int(first) == int(logits.argmax(-1))


def greedy_ft(host, prompt, count):
    """The reference's fused_ft_kernel decode (generation.py:77-140 with
    fused_ft_kernel=True): prefill writes the FT caches, every decode step
    rotates, appends and attends in one FT call."""
    from hexgen2_amd.generation import InferenceParams
    params = InferenceParams(max_sequence_len=len(prompt) + count, max_batch_size=1, fused_ft_kernel=True)
    logits = host.forward(torch.tensor([prompt], device="cuda"), params)
    token = int(logits.argmax(-1))
    tokens = [token]
    params.sequence_len_offset = len(prompt)
    for _ in range(count - 1):
        logits = host.forward(torch.tensor([[token]], device="cuda"), params)
        token = int(logits.argmax(-1))
        tokens.append(token)
        params.sequence_len_offset += 1
    assert isinstance(params.key_value_memory_dict[0], tuple)  # the FT K/V pair
    return tokens


@pytest.mark.parametrize("dtype", ["float16", "bfloat16", "float32"])
def test_ft_decode_tokens_match_reference(device, dtype):
    from hexgen2_amd.llama import LlamaHost
    host = LlamaHost.load(GOLDEN / "fixture_seed17", "cuda", getattr(torch, dtype))
    for case in GREEDY["fixture_seed17"]:
        print(f"ft fixture {dtype} prompt={case['prompt']}", flush=True)
        assert greedy_ft(host, case["prompt"], case["max_new_tokens"]) == case["reference_gpu_fp16_tokens"]
    if dtype == "float32":
        tiny = LlamaHost.load(GOLDEN / "tiny_llama", "cuda", torch.float32)
        case = GREEDY["tiny_llama"][0]
        assert greedy_ft(tiny, case["prompt"], case["max_new_tokens"]) == case["hf_fp32_tokens"]
