"""Ragged decode batches through the reference's call sites.

The reference keeps one ``sequence_len_offset`` for the whole batch on the
standard cache layout (hexgen/hexgen_core/modules/mha.py:276-279) and reads
per-sample positions from ``InferenceParams.lengths_per_sample``
(generation.py:30) only on the FT path (mha.py:327-328).  Here the same field
drives ``_update_kv_cache`` (append at each sample's own position),
``FlashCrossAttention`` (each row attends its own key count) and the fused
``update_and_attend``.  Checked against the oracle: the append bit-exact, the
attention within the dtype's tolerance (fp16 2e-3, bf16 8e-3, fp32 2e-5
max-abs against float64), over several steps; and at model level a ragged
batch of 8 prompts decoded together gives the tokens each prompt gets when
decoded alone, with logits within the reference validator's
``allclose(atol=0.03, rtol=0.03)`` (hexgen2/validate.py:43).
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from hexgen2_amd import ops
from hexgen2_amd.generation import InferenceParams
from hexgen2_amd.llama import LlamaHost
from hexgen2_amd.mha import FlashCrossAttention, _update_kv_cache, update_and_attend
from oracle import kv_oracle as oracle

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
TOL = {torch.float16: 2e-3, torch.bfloat16: 8e-3, torch.float32: 2e-5}
INT_VIEW = {torch.float16: torch.int16, torch.bfloat16: torch.int16, torch.float32: torch.int32}


def bits(t):
    return t.detach().cpu().contiguous().view(INT_VIEW[t.dtype]).numpy()


def f64(t):
    return t.detach().cpu().double().numpy()


@pytest.mark.parametrize("dtype,hq,hkv,d", [(torch.float16, 32, 4, 64), (torch.bfloat16, 32, 8, 128),
                                            (torch.float32, 4, 4, 16), (torch.bfloat16, 8, 1, 128)])
@pytest.mark.parametrize("fused", [False, True])
def test_ragged_steps_through_call_sites(device, dtype, hq, hkv, d, fused):
    lens = [0, 1, 17, 300, 64, 1025, 5, 700]
    steps, cap = 3, 1100
    print(f"ragged call sites {dtype} {hq}/{hkv}/{d} fused={fused}", flush=True)
    g = torch.Generator(device=device).manual_seed(21)
    cache = torch.randn((len(lens), cap, 2, hkv, d), generator=g, device=device).to(dtype)
    lengths = torch.tensor(lens, dtype=torch.int32, device=device)
    params = InferenceParams(max_sequence_len=cap, max_batch_size=len(lens), sequence_len_offset=max(lens),
                             key_value_memory_dict={0: cache}, lengths_per_sample=lengths)
    attn = FlashCrossAttention(causal=True)
    cur = list(lens)
    for step in range(steps):
        q = torch.randn((len(lens), 1, hq, d), generator=g, device=device).to(dtype)
        kv = torch.randn((len(lens), 1, 2, hkv, d), generator=g, device=device).to(dtype)
        before = bits(cache)
        if fused:
            out = update_and_attend(q, kv, params, 0)
        else:
            view = _update_kv_cache(kv, params, 0)
            assert view.shape[1] == params.sequence_len_offset + 1
            out = attn(q, view, causal=False)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(cache), oracle.append(before, bits(kv[:, 0]), cur))
        ref = oracle.attend(f64(q), f64(cache), [n + 1 for n in cur])
        err = float(np.abs(f64(out) - ref).max())
        assert err <= TOL[dtype], f"step {step}: max-abs {err}"
        lengths += 1
        params.sequence_len_offset += 1
        cur = [n + 1 for n in cur]


def test_ragged_sub_batch_offset(device):
    # batch_size_offset selects lengths_per_sample[3:7] and cache rows 3..6
    lens = [9, 40, 3, 200, 0, 77, 150, 31]
    cap, dtype = 256, torch.bfloat16
    g = torch.Generator(device=device).manual_seed(22)
    cache = torch.randn((8, cap, 2, 8, 128), generator=g, device=device).to(dtype)
    lengths = torch.tensor(lens, dtype=torch.int32, device=device)
    params = InferenceParams(max_sequence_len=cap, max_batch_size=8, sequence_len_offset=max(lens),
                             batch_size_offset=3, key_value_memory_dict={0: cache}, lengths_per_sample=lengths)
    q = torch.randn((4, 1, 32, 128), generator=g, device=device).to(dtype)
    kv = torch.randn((4, 1, 2, 8, 128), generator=g, device=device).to(dtype)
    before = bits(cache)
    out = FlashCrossAttention()(q, _update_kv_cache(kv, params, 0), causal=False)
    torch.cuda.synchronize()
    want = before.copy()
    want[3:7] = oracle.append(before[3:7], bits(kv[:, 0]), lens[3:7])
    np.testing.assert_array_equal(bits(cache), want)
    ref = oracle.attend(f64(q), f64(cache[3:7]), [n + 1 for n in lens[3:7]])
    assert np.abs(f64(out) - ref).max() <= TOL[dtype]


def test_explicit_seqlens_k(device):
    # FlashCrossAttention's seqlens_k keyword over a plain padded cache view
    g = torch.Generator(device=device).manual_seed(23)
    cache = torch.randn((3, 64, 2, 2, 64), generator=g, device=device).to(torch.float16)
    q = torch.randn((3, 1, 8, 64), generator=g, device=device).to(torch.float16)
    seqlens = torch.tensor([5, 64, 1], dtype=torch.int32, device=device)
    out = FlashCrossAttention()(q, cache, causal=False, seqlens_k=seqlens)
    ref = oracle.attend(f64(q), f64(cache), [5, 64, 1])
    assert np.abs(f64(out) - ref).max() <= TOL[torch.float16]


def _decode_alone(host, ids, new_tokens, fused):
    """Batch-1 prefill + greedy decode: (tokens, per-step logits, live cache
    per layer [1, L, 2, Hkv, D])."""
    state = InferenceParams(max_sequence_len=len(ids) + new_tokens)
    logits = [host.forward(torch.tensor([ids], device=host.device), state)]
    live = [state.key_value_memory_dict[i][:, :len(ids)].clone() for i in range(len(host.layers))]
    state.sequence_len_offset = len(ids)
    tokens = [int(logits[-1].argmax(-1))]
    for _ in range(new_tokens - 1):
        logits.append(host.forward(torch.tensor([[tokens[-1]]], device=host.device), state,
                                   fused_append=fused))
        state.sequence_len_offset += 1
        tokens.append(int(logits[-1].argmax(-1)))
    return tokens, [x[0].float() for x in logits], live


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("fused", [False, True])
def test_ragged_batch_decode_equals_decoding_alone(device, dtype, fused):
    host = LlamaHost.load(GOLDEN / "fixture_seed17", device, dtype)
    rng = np.random.default_rng(5)
    lens = [1, 9, 4, 23, 2, 16, 7, 30]
    prompts = [rng.integers(0, host.shape.vocab_size, n).tolist() for n in lens]
    new_tokens = 6
    print(f"ragged model decode {dtype} fused={fused} lens={lens}", flush=True)
    alone = [_decode_alone(host, ids, new_tokens, fused) for ids in prompts]

    # The per-sequence live caches, packed back to back (the reference's
    # per-request packets in send order), unpacked into one ragged batch.
    n_layers = len(host.layers)
    packed = torch.cat([torch.stack([c[0] for c in live], 0) for _, _, live in alone], dim=1)
    cap = max(lens) + new_tokens
    row = alone[0][2][0].shape[2:]
    decode = torch.empty((n_layers, len(lens), cap, *row), dtype=dtype, device=device)
    ops.unpack_live(packed, decode, lens)
    lengths = torch.tensor(lens, dtype=torch.int32, device=device)
    params = InferenceParams(max_sequence_len=cap, max_batch_size=len(lens), sequence_len_offset=max(lens),
                             key_value_memory_dict={i: decode[i] for i in range(n_layers)},
                             lengths_per_sample=lengths)
    token = torch.tensor([t[0][0] for t in alone], device=device)
    for step in range(1, new_tokens):
        logits = host.forward(token[:, None], params, fused_append=fused).float()
        params.sequence_len_offset += 1
        lengths += 1
        token = logits.argmax(-1)
        for b, (tokens, want_logits, _) in enumerate(alone):
            assert int(token[b]) == tokens[step], (b, step)
            torch.testing.assert_close(logits[b], want_logits[step], atol=0.03, rtol=0.03)


@pytest.mark.parametrize("fused", [False, True])
def test_lengths_past_the_offset_are_reported(device, fused):
    """lengths_per_sample[b] > sequence_len_offset breaks the ragged contract
    (the attended view ends at the offset).  The reference would assert on
    the host (mha.py:281-282); here every kernel exits normally, row b is cut
    to the view (so its own new key is missed) and the status word reports
    it: mha.check_kv_status raises ValueError at the caller's next check.
    In-contract steps before and after leave it clear."""
    from hexgen2_amd.mha import check_kv_status

    dtype, hq, hkv, d = torch.float16, 8, 2, 64
    g = torch.Generator(device=device).manual_seed(5)
    cap = 64
    cache = torch.randn((3, cap, 2, hkv, d), generator=g, device=device).to(dtype)
    ops.device_status()  # start clear

    def step(lens, offset):
        lengths = torch.tensor(lens, dtype=torch.int32, device=device)
        params = InferenceParams(max_sequence_len=cap, max_batch_size=3, sequence_len_offset=offset,
                                 key_value_memory_dict={0: cache}, lengths_per_sample=lengths)
        q = torch.randn((3, 1, hq, d), generator=g, device=device).to(dtype)
        kv = torch.randn((3, 1, 2, hkv, d), generator=g, device=device).to(dtype)
        if fused:
            out = update_and_attend(q, kv, params, 0)
        else:
            out = FlashCrossAttention(causal=True)(q, _update_kv_cache(kv, params, 0), causal=False)
        torch.cuda.synchronize()
        return out

    step([5, 9, 12], 12)
    check_kv_status()  # in contract: nothing raised
    out = step([5, 30, 12], 12)  # row 1 sits past the offset
    assert torch.isfinite(out.float()).all()
    with pytest.raises(ValueError, match="exceeded the attended view"):
        check_kv_status()
    step([6, 10, 13], 13)
    check_kv_status()  # the check cleared the flag


def test_prompt_step_ignores_lengths_per_sample(device):
    """At sequence_len_offset 0 (the prompt) _update_kv_cache writes at the
    offset even when lengths_per_sample is set -- the reference's generation
    loop fills it with the prompt lengths before the prompt's forward
    (generation.py:380) -- so a one-token prompt lands at position 0."""
    dtype, hkv, d = torch.float16, 2, 64
    cache = torch.zeros((2, 16, 2, hkv, d), dtype=dtype, device=device)
    params = InferenceParams(max_sequence_len=16, max_batch_size=2, sequence_len_offset=0,
                             key_value_memory_dict={0: cache},
                             lengths_per_sample=torch.tensor([1, 1], dtype=torch.int32, device=device))
    kv = torch.ones((2, 1, 2, hkv, d), dtype=dtype, device=device)
    view = _update_kv_cache(kv, params, 0)
    torch.cuda.synchronize()
    assert view.shape[1] == 1
    assert (cache[:, 0] == 1).all() and (cache[:, 1:] == 0).all()
