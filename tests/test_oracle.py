"""Pins the CPU oracle (oracle/kv_oracle.py) before it is trusted as the checker.

Pack/unpack/append: element-by-element loops, the round-trip and untouched-row
invariants, and the handoff sizes the reference recorded.  Attention: closed
forms, a scalar-loop restatement, and torch's scaled_dot_product_attention in
float64 as an independent library routine.
"""
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import kv_oracle as oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def _caches(rng, n_layers, batch, cap, hkv=2, d=3):
    return [rng.standard_normal((batch, cap, 2, hkv, d)).astype(np.float32) for _ in range(n_layers)]


@pytest.mark.parametrize("lens", [[4], [0, 3, 5], [5, 0, 0, 1], [1, 1, 1]])
def test_pack_matches_elementwise_loop(lens):
    rng = np.random.default_rng(0)
    caches = _caches(rng, 3, len(lens), 5)
    packed = oracle.pack(caches, lens)
    assert packed.shape == (3, sum(lens), 2, 2, 3)
    for l in range(3):
        r = 0
        for b, n in enumerate(lens):
            for s in range(n):
                for k in range(2):
                    for h in range(2):
                        for i in range(3):
                            assert packed[l, r, k, h, i] == caches[l][b, s, k, h, i]
                r += 1
        assert r == sum(lens)


def test_pack_batch1_equals_reference_slice():
    # model.py:81: t[:, :L].contiguous() -- batch-1 packing is the plain slice
    rng = np.random.default_rng(1)
    caches = _caches(rng, 2, 1, 9)
    packed = oracle.pack(caches, [6])
    for l in range(2):
        np.testing.assert_array_equal(packed[l], caches[l][0, :6])


def test_unpack_roundtrip_and_untouched_rows():
    rng = np.random.default_rng(2)
    lens = [3, 0, 7, 1]
    src = _caches(rng, 2, 4, 8)
    packed = oracle.pack(src, lens)
    sentinel = [np.full_like(c, -7.5) for c in src]
    out = oracle.unpack(packed, sentinel, lens)
    for l in range(2):
        for b, n in enumerate(lens):
            np.testing.assert_array_equal(out[l][b, :n], src[l][b, :n])
            assert (out[l][b, n:] == -7.5).all()
    # inputs are not modified
    assert all((s == -7.5).all() for s in sentinel)


def test_append_writes_exactly_one_row_per_sequence():
    rng = np.random.default_rng(3)
    cache = rng.standard_normal((3, 6, 2, 1, 4)).astype(np.float32)
    kv = rng.standard_normal((3, 2, 1, 4)).astype(np.float32)
    out = oracle.append(cache, kv, [0, 5, 2])
    for b, pos in enumerate([0, 5, 2]):
        np.testing.assert_array_equal(out[b, pos], kv[b])
        for s in range(6):
            if s != pos:
                np.testing.assert_array_equal(out[b, s], cache[b, s])
    with pytest.raises(ValueError):
        oracle.append(cache, kv, [0, 6, 0])


def test_packet_bytes_match_reference_evidence():
    # kv_packet_bytes recorded by the reference pilot = int64 token + live KV
    cases = json.loads((GOLDEN / "packet_bytes.json").read_text())["cases"]
    assert len(cases) == 7
    for c in cases:
        assert oracle.kv_packet_bytes(c["layers"], c["prompt_tokens"], c["kv_heads"],
                                      c["head_dim"], c["elem_bytes"]) == c["kv_packet_bytes"]
        # and the same figure through the header payload accounting
        shapes = [([1], "torch.int64")] + [([1, c["prompt_tokens"], 2, c["kv_heads"], c["head_dim"]],
                                            "torch.float16")] * c["layers"]
        assert oracle.packet_payload_bytes(shapes) == c["kv_packet_bytes"]
    # pack output size agrees with the same accounting
    c = cases[5]  # TinyLlama, 82-token prompt
    caches = [np.zeros((1, 90, 2, 4, 64), np.float16)] * 2
    assert oracle.pack(caches, [82]).nbytes == 2 * 82 * 1024


def _rand_attn(rng, batch, sq, hq, hkv, d, cap):
    q = rng.standard_normal((batch, sq, hq, d))
    cache = rng.standard_normal((batch, cap, 2, hkv, d))
    return q, cache


def test_attend_single_key_returns_its_value():
    rng = np.random.default_rng(4)
    q, cache = _rand_attn(rng, 2, 1, 8, 2, 16, 4)
    out = oracle.attend(q, cache, [1, 1])
    for b in range(2):
        for h in range(8):
            np.testing.assert_allclose(out[b, 0, h], cache[b, 0, 1, h // 4], rtol=0, atol=1e-15)


def test_attend_equal_keys_or_zero_query_average_values():
    rng = np.random.default_rng(5)
    q, cache = _rand_attn(rng, 1, 1, 4, 4, 8, 10)
    cache[:, :, 0] = cache[:, :1, 0]  # every key equal
    out = oracle.attend(q, cache, [7])
    np.testing.assert_allclose(out[0, 0], cache[0, :7, 1].mean(axis=0), atol=1e-12)
    q[:] = 0
    q2, cache2 = _rand_attn(rng, 1, 1, 4, 4, 8, 10)
    out = oracle.attend(np.zeros_like(q2), cache2, [10])
    np.testing.assert_allclose(out[0, 0], cache2[0, :, 1].mean(axis=0), atol=1e-12)


def test_attend_dominant_key_selects_its_value():
    rng = np.random.default_rng(6)
    q, cache = _rand_attn(rng, 1, 1, 2, 1, 16, 9)
    cache[0, 5, 0, 0] = q[0, 0, 0] * 100.0  # huge score for q head 0 only
    out = oracle.attend(q, cache, [9])
    np.testing.assert_allclose(out[0, 0, 0], cache[0, 5, 1, 0], atol=1e-12)


def test_attend_matches_scalar_loop_and_grouping():
    rng = np.random.default_rng(7)
    q, cache = _rand_attn(rng, 2, 1, 6, 2, 5, 7)
    lens = [7, 3]
    np.testing.assert_allclose(oracle.attend(q, cache, lens), oracle.attend_loop(q, cache, lens),
                               rtol=1e-12, atol=1e-12)
    # GQA with group g equals MHA over the head-repeated cache
    mha_cache = np.repeat(cache, 3, axis=3)
    np.testing.assert_allclose(oracle.attend(q, cache, lens), oracle.attend(q, mha_cache, lens),
                               rtol=0, atol=1e-15)


@pytest.mark.parametrize("causal", [False, True])
def test_attend_matches_torch_sdpa_fp64(causal):
    rng = np.random.default_rng(8)
    batch, sq, hq, hkv, d = 2, 5 if causal else 1, 8, 2, 32
    lens = [5, 9] if causal else [13, 4]
    q, cache = _rand_attn(rng, batch, sq, hq, hkv, d, 16)
    out = oracle.attend(q, cache, lens, causal=causal, softmax_scale=0.3)
    for b in range(batch):
        n = lens[b]
        k = torch.from_numpy(np.repeat(cache[b, :n, 0], hq // hkv, axis=1)).permute(1, 0, 2)
        v = torch.from_numpy(np.repeat(cache[b, :n, 1], hq // hkv, axis=1)).permute(1, 0, 2)
        qq = torch.from_numpy(q[b]).permute(1, 0, 2)
        mask = None
        if causal:  # bottom-right aligned triangle
            mask = torch.arange(n)[None, :] <= (n - sq + torch.arange(sq))[:, None]
        ref = torch.nn.functional.scaled_dot_product_attention(qq, k, v, attn_mask=mask, scale=0.3)
        np.testing.assert_allclose(out[b], ref.permute(1, 0, 2).numpy(), rtol=1e-10, atol=1e-12)


def test_attend_causal_prefill_equals_reference_triangle():
    # With Sq == Sk, query t sees keys <= t: CrossAttention's triu(-10000, 1) mask (mha.py:238-241)
    rng = np.random.default_rng(9)
    q, cache = _rand_attn(rng, 1, 6, 2, 2, 4, 6)
    out = oracle.attend(q, cache, [6], causal=True)
    for t in range(6):
        row = oracle.attend(q[:, t:t + 1], cache, [t + 1])
        np.testing.assert_allclose(out[:, t], row[:, 0], atol=1e-14)


def test_attend_scale_default_is_inverse_sqrt_head_dim():
    rng = np.random.default_rng(10)
    q, cache = _rand_attn(rng, 1, 1, 2, 2, 16, 5)
    np.testing.assert_allclose(oracle.attend(q, cache, [5]),
                               oracle.attend(q, cache, [5], softmax_scale=1 / math.sqrt(16)), atol=0)


# ---------------------------------------------------------- legacy formats ---
# Pinned against the library routines the reference calls (torch.cat,
# torch.nn.functional.pad with the reference's own pad tuple) and against the
# inverses (slicing the result back into its parts).

def _rand(rng, shape):
    return rng.standard_normal(shape).astype(np.float32)


def test_flat_concat_is_torch_cat_of_flattened_and_splits_back():
    rng = np.random.default_rng(1)
    base = _rand(rng, (2, 6, 2, 3, 4))
    tensors = [base[:, :5], _rand(rng, (1, 3, 2, 3, 4)), base.transpose(1, 0, 2, 3, 4), _rand(rng, (0, 4))]
    flat = oracle.flat_concat(tensors)
    want = torch.cat([torch.from_numpy(np.ascontiguousarray(t)).flatten() for t in tensors]).numpy()
    np.testing.assert_array_equal(flat, want)
    for got, t in zip(oracle.flat_split(flat, [t.shape for t in tensors]), tensors):
        np.testing.assert_array_equal(got, t)


def test_flat_packet_of_reference_example_shapes():
    # kv_cache_communication.py:75-84: 32 layers of [1, 150, 2, 32, 128]
    shapes = [(1, 150, 2, 32, 128)] * 32
    assert sum(math.prod(s) for s in shapes) == 32 * 150 * 2 * 32 * 128
    flat = oracle.flat_concat([np.full(s[1:2], i, dtype=np.int16) for i, s in enumerate(shapes)])
    assert flat.shape == (32 * 150,) and flat[150 * 7] == 7


def test_batch_pad_is_reference_pad_then_cat():
    rng = np.random.default_rng(2)
    reqs = [_rand(rng, (1, 5, 2, 3, 4)), _rand(rng, (3, 2, 2, 3, 4)), _rand(rng, (2, 0, 2, 3, 4)),
            _rand(rng, (1, 7, 2, 3, 4))]
    got = oracle.batch_pad(reqs)
    # kv_cache_batch.py:17-22 verbatim semantics: F.pad(t, (0,0,0,0,0,0,0,pad)) then cat(dim=0)
    import torch.nn.functional as F
    parts = []
    for r in reqs:
        t = torch.from_numpy(r)
        pad = 7 - t.size(1)
        parts.append(F.pad(t, (0, 0, 0, 0, 0, 0, 0, pad), "constant", 0) if pad > 0 else t)
    np.testing.assert_array_equal(got, torch.cat(parts, dim=0).numpy())
    # inverse: each request comes back from its rows; the padding is zero
    row = 0
    for r in reqs:
        b, s = r.shape[:2]
        np.testing.assert_array_equal(got[row:row + b, :s], r)
        assert not got[row:row + b, s:].any()
        row += b
    assert got.shape == (7, 7, 2, 3, 4)


def test_batch_pad_reference_example_shapes():
    # kv_cache_batch.py:38-44: [1, 150, ...] and [1, 128, ...] -> [2, 150, ...]
    a, b = np.ones((1, 150, 2, 1, 2), np.float32), np.ones((1, 128, 2, 1, 2), np.float32)
    got = oracle.batch_pad([a, b])
    assert got.shape == (2, 150, 2, 1, 2)
    assert got[1, 127].all() and not got[1, 128:].any() and got[0].all()
    with pytest.raises(ValueError):
        oracle.batch_pad([a], max_rows=100)


@pytest.mark.parametrize("dim", [3, -2, 0, 1, 4])
def test_concat_dim_is_torch_cat_and_splits_back(dim):
    rng = np.random.default_rng(3)
    heads = [1, 3, 2]
    shards = []
    for h in heads:
        shape = [2, 4, 2, 2, 5]
        shape[dim % 5] = h
        shards.append(_rand(rng, tuple(shape)))
    got = oracle.concat_dim(shards, dim)
    np.testing.assert_array_equal(got, torch.cat([torch.from_numpy(s) for s in shards], dim=dim).numpy())
    pieces = np.split(got, np.cumsum(heads)[:-1], axis=dim)
    for p, s in zip(pieces, shards):
        np.testing.assert_array_equal(p, s)


def test_concat_dim_default_is_the_kv_head_dim():
    # tensor_parallel_dim_concat.py:9: dim=3 of [B, S, 2, H, D] joins the heads,
    # so kv head h of the result is shard h // Hs's head h % Hs
    rng = np.random.default_rng(4)
    shards = [_rand(rng, (2, 3, 2, 2, 4)) for _ in range(4)]
    got = oracle.concat_dim(shards)
    assert got.shape == (2, 3, 2, 8, 4)
    for h in range(8):
        np.testing.assert_array_equal(got[:, :, :, h], shards[h // 2][:, :, :, h % 2])


# ------------------------------------------------------ FasterTransformer ---


@pytest.mark.parametrize("dtype,pack", [(np.float16, 8), (np.float32, 4)])
def test_ft_layout_is_the_reference_rearrange(dtype, pack):
    """ft_layout == einops.rearrange with the patterns of mha.py:296-298."""
    import einops
    rng = np.random.default_rng(3)
    cache = rng.standard_normal((2, 7, 2, 3, 16)).astype(dtype)
    k, v = oracle.ft_layout(cache, pack)
    t = torch.from_numpy(cache)
    k_ref = einops.rearrange(t[:, :, 0], "b s h (d packsize) -> b h d s packsize", packsize=pack).contiguous()
    v_ref = einops.rearrange(t[:, :, 1], "b s h d -> b h s d").contiguous()
    assert k.shape == (2, 3, 16 // pack, 7, pack) and v.shape == (2, 3, 7, 16)
    np.testing.assert_array_equal(k, k_ref.numpy())
    np.testing.assert_array_equal(v, v_ref.numpy())
    np.testing.assert_array_equal(oracle.ft_unlayout(k, v), cache)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16", "float32"])
def test_round_to_matches_torch_casts(dtype):
    rng = np.random.default_rng(4)
    x = rng.standard_normal(4096) * 10.0 ** rng.integers(-3, 4, 4096)
    got = oracle.round_to(x, dtype)
    want = torch.from_numpy(x.astype(np.float32)).to(getattr(torch, dtype)).to(torch.float64).numpy()
    np.testing.assert_array_equal(got, want)


def test_rotary_closed_forms():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 16))
    for neox in (True, False):
        np.testing.assert_array_equal(oracle.rotary(x, 0, 16, 10000.0, neox), x)  # position 0
        np.testing.assert_array_equal(oracle.rotary(x, 9, 0, 10000.0, neox), x)   # no rotary dims
        y = oracle.rotary(x, 37, 8, 500.0, neox)
        np.testing.assert_array_equal(y[:, 8:], x[:, 8:])                         # beyond rot_dim
        pairs = [(j, j + 4) if neox else (2 * j, 2 * j + 1) for j in range(4)]
        for i0, i1 in pairs:                                                      # each pair keeps its norm
            np.testing.assert_allclose(np.hypot(y[:, i0], y[:, i1]), np.hypot(x[:, i0], x[:, i1]), rtol=1e-12)
    # a 2-vector turns by pos radians (pair 0 has frequency 1)
    v = np.array([1.0, 0.0])
    np.testing.assert_allclose(oracle.rotary(v, 3, 2, 10000.0, True), [math.cos(3), math.sin(3)], atol=1e-15)


@pytest.mark.parametrize("pos,rot_dim,base", [(1, 64, 10000.0), (1234, 64, 10000.0), (77, 32, 500000.0)])
def test_rotary_neox_matches_transformers_llama(pos, rot_dim, base):
    """The GPT-NeoX form equals transformers' Llama apply_rotary_pos_emb
    (rotate_half) on the rotated dimensions; the GPT-J form equals it after
    gathering each (2j, 2j+1) pair into (j, j + rot_dim/2)."""
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    rng = np.random.default_rng(pos)
    q = rng.standard_normal((1, 2, 1, rot_dim))
    inv_freq = 1.0 / (base ** (torch.arange(0, rot_dim, 2, dtype=torch.float64) / rot_dim))
    freqs = pos * inv_freq
    emb = torch.cat((freqs, freqs))[None, None]
    qt = torch.from_numpy(q)
    q_hf, _ = apply_rotary_pos_emb(qt, qt, emb.cos(), emb.sin())
    np.testing.assert_allclose(oracle.rotary(q, pos, rot_dim, base, True), q_hf.numpy(), rtol=1e-12, atol=1e-12)
    perm = np.concatenate([np.arange(0, rot_dim, 2), np.arange(1, rot_dim, 2)])  # pairs -> halves
    gptj = oracle.rotary(q, pos, rot_dim, base, False)
    np.testing.assert_allclose(gptj[..., perm], oracle.rotary(q[..., perm], pos, rot_dim, base, True),
                               rtol=1e-12, atol=1e-12)


def test_ft_decode_without_rotary_is_append_then_attend():
    rng = np.random.default_rng(6)
    batch, cap, hkv, hq, d = 3, 12, 2, 4, 8
    cache = rng.standard_normal((batch, cap, 2, hkv, d)).astype(np.float32)
    q = rng.standard_normal((batch, hq, d)).astype(np.float32)
    kv_new = rng.standard_normal((batch, 2, hkv, d)).astype(np.float32)
    positions = [0, 5, 11]
    k_ft, v_ft = oracle.ft_layout(cache, 4)
    out, k2, v2 = oracle.ft_decode(q, kv_new[:, 0], kv_new[:, 1], k_ft, v_ft, positions)
    appended = oracle.append(cache, kv_new, positions)
    want = oracle.attend(q[:, None], appended, [p + 1 for p in positions])[:, 0]
    np.testing.assert_allclose(out, want, rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(oracle.ft_unlayout(k2, v2), appended)
