"""GPU parity of the FasterTransformer (FT) cache path: hexkv_ft_store and
hexkv_ft_attend (hexgen/hexgen_core/modules/mha.py:289-337).

ft_store is a bit copy: compared as integer views with oracle.ft_layout, and
positions past the stored ones keep their sentinel.  ft_attend against
oracle.ft_decode in float64 with the tolerances of hexkv_attend (fp16 2e-3,
bf16 8e-3, fp32 2e-5); the appended V bit-exact, the appended (rotated) K to
within the rounding of the dtype (the kernel turns it in fp32, the oracle in
float64, and both then round).  Without rotation the FT path equals
hexkv_attend's VALU kernel on the same data in the standard layout, bit for
bit: the arithmetic is the same, only the addresses differ.  The
ft_attention extension the reference calls is not vendored, so its own
outputs pin nothing here; the rotary form is pinned on the CPU against
transformers' Llama rotary (tests/test_oracle.py).
"""
import numpy as np
import pytest
import torch

from hexgen2_amd import generation, mha, ops
from oracle import kv_oracle as oracle

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-3, torch.bfloat16: 8e-3, torch.float32: 2e-5}
# Appended K: the rounding of the dtype (fp16, bf16), or for fp32 the fp32
# turn itself (x0 cos - x1 sin, about 2^-23 of |x|).
REL = {torch.float16: 2e-3, torch.bfloat16: 8e-3, torch.float32: 1e-6}
ATOL_K = {torch.float16: 2e-5, torch.bfloat16: 8e-5, torch.float32: 5e-7}
INT_VIEW = {torch.float16: torch.int16, torch.bfloat16: torch.int16, torch.float32: torch.int32}
NAME = {torch.float16: "float16", torch.bfloat16: "bfloat16", torch.float32: "float32"}


def bits(t):
    return t.detach().cpu().contiguous().view(INT_VIEW[t.dtype]).numpy()


def f64(t):
    return t.detach().cpu().double().numpy()


def to_device(int_array, dtype, device):
    return torch.from_numpy(np.ascontiguousarray(int_array)).view(dtype).to(device)


@pytest.mark.parametrize("dtype,batch,seq,cap,hkv,d", [
    (torch.float16, 2, 5, 9, 3, 64),
    (torch.bfloat16, 3, 129, 200, 8, 128),
    (torch.float32, 2, 7, 7, 2, 16),
    (torch.bfloat16, 1, 1, 4, 1, 256),
    (torch.float16, 2, 0, 3, 2, 32),
    (torch.bfloat16, 2, 600, 640, 3, 32),  # two full 256-position tiles + 88; 12 chunks: 8 + 4
    (torch.float32, 1, 300, 301, 1, 16),   # 4 chunks per row: one partial chunk tile
])
def test_ft_store_is_the_reference_layout(device, dtype, batch, seq, cap, hkv, d):
    print(f"ft_store {dtype} b={batch} s={seq} cap={cap} h={hkv} d={d}", flush=True)
    g = torch.Generator(device=device).manual_seed(11)
    kv = torch.randn((batch, seq, 2, hkv, d), generator=g, device=device).to(dtype)
    k_shape, v_shape = ops.ft_cache_shapes(batch, hkv, cap, d, dtype)
    k_cache = torch.full(k_shape, -7.25, dtype=dtype, device=device)
    v_cache = torch.full(v_shape, -7.25, dtype=dtype, device=device)
    ops.ft_store(kv, k_cache, v_cache)
    torch.cuda.synchronize()
    sentinel = bits(torch.tensor([-7.25], dtype=dtype))[0]
    k_ref, v_ref = oracle.ft_layout(bits(kv), ops.ft_pack(dtype))
    np.testing.assert_array_equal(bits(k_cache)[:, :, :, :seq], k_ref)
    np.testing.assert_array_equal(bits(v_cache)[:, :, :seq], v_ref)
    assert (bits(k_cache)[:, :, :, seq:] == sentinel).all() and (bits(v_cache)[:, :, seq:] == sentinel).all()


def test_ft_store_from_a_cache_view_into_a_batch_slice(device):
    """The conversion of mha.py:295-299: the source is the live prefix of a
    [B, S, 2, H, D] cache (strided); the target is a batch slice."""
    dtype, batch, cap, hkv, d = torch.bfloat16, 4, 40, 2, 64
    g = torch.Generator(device=device).manual_seed(12)
    full = torch.randn((batch, cap, 2, hkv, d), generator=g, device=device).to(dtype)
    src = full[1:3, :17]
    k_shape, v_shape = ops.ft_cache_shapes(batch, hkv, cap, d, dtype)
    k_cache = torch.zeros(k_shape, dtype=dtype, device=device)
    v_cache = torch.zeros(v_shape, dtype=dtype, device=device)
    ops.ft_store(src, k_cache[1:3], v_cache[1:3])
    torch.cuda.synchronize()
    k_ref, v_ref = oracle.ft_layout(bits(src), ops.ft_pack(dtype))
    np.testing.assert_array_equal(bits(k_cache)[1:3, :, :, :17], k_ref)
    np.testing.assert_array_equal(bits(v_cache)[1:3, :, :17], v_ref)
    assert (bits(k_cache)[[0, 3]] == 0).all() and (bits(k_cache)[1:3, :, :, 17:] == 0).all()
    assert (bits(v_cache)[[0, 3]] == 0).all() and (bits(v_cache)[1:3, :, 17:] == 0).all()


def test_ft_store_from_an_unaligned_view(device):
    """A source that is not 16-byte aligned takes the span-engine path."""
    dtype, batch, seq, cap, hkv, d = torch.float16, 2, 33, 40, 2, 64
    g = torch.Generator(device=device).manual_seed(13)
    flat = torch.randn(batch * seq * 2 * hkv * d + 1, generator=g, device=device).to(dtype)
    kv = flat[1:].view(batch, seq, 2, hkv, d)
    assert kv.data_ptr() % 16
    k_shape, v_shape = ops.ft_cache_shapes(batch, hkv, cap, d, dtype)
    k_cache = torch.zeros(k_shape, dtype=dtype, device=device)
    v_cache = torch.zeros(v_shape, dtype=dtype, device=device)
    ops.ft_store(kv, k_cache, v_cache)
    torch.cuda.synchronize()
    k_ref, v_ref = oracle.ft_layout(bits(kv), ops.ft_pack(dtype))
    np.testing.assert_array_equal(bits(k_cache)[:, :, :, :seq], k_ref)
    np.testing.assert_array_equal(bits(v_cache)[:, :, :seq], v_ref)
    assert (bits(k_cache)[:, :, :, seq:] == 0).all() and (bits(v_cache)[:, :, seq:] == 0).all()


def ft_case(device, dtype, hq, hkv, d, positions, cap, seed):
    g = torch.Generator(device=device).manual_seed(seed)
    batch = len(positions)
    cache = torch.randn((batch, cap, 2, hkv, d), generator=g, device=device).to(dtype)
    q = torch.randn((batch, hq, d), generator=g, device=device).to(dtype)
    new = torch.randn((batch, 2, hkv, d), generator=g, device=device).to(dtype)
    k_int, v_int = oracle.ft_layout(bits(cache), ops.ft_pack(dtype))
    return cache, q, new, to_device(k_int, dtype, device), to_device(v_int, dtype, device)


FT_GEOMETRIES = [
    (8, 2, 128, torch.bfloat16),   # group 4
    (32, 8, 128, torch.bfloat16),  # Llama-3-8B
    (8, 1, 128, torch.float16),    # group 8
    (4, 4, 64, torch.float16),     # MHA
    (6, 2, 64, torch.float16),     # group 3
    (4, 2, 16, torch.float32),     # fp32, pack 4
    (4, 2, 256, torch.bfloat16),   # head_dim 256
]


@pytest.mark.parametrize("hq,hkv,d,dtype", FT_GEOMETRIES)
@pytest.mark.parametrize("rot", ["none", "neox", "gptj", "neox-half"])
def test_ft_attend_matches_oracle(device, hq, hkv, d, dtype, rot):
    positions = [0, 5, 130, 1000]
    cap = 1100
    rot_dim = {"none": 0, "neox": d, "gptj": d, "neox-half": d // 2}[rot]
    neox = rot != "gptj"
    base = 10000.0 if rot != "neox-half" else 500000.0
    print(f"ft_attend {dtype} hq={hq} hkv={hkv} d={d} rot={rot}", flush=True)
    cache, q, new, k_ft, v_ft = ft_case(device, dtype, hq, hkv, d, positions, cap, 21)
    pos = torch.tensor(positions, dtype=torch.int32, device=device)
    k_before, v_before = bits(k_ft), bits(v_ft)
    out = ops.ft_attend(q, new[:, 0], new[:, 1], k_ft, v_ft, max_position=max(positions), positions=pos,
                        rotary_dim=rot_dim, rotary_base=base, rotary_neox=neox)
    torch.cuda.synchronize()
    ref, k2, v2 = oracle.ft_decode(f64(q), f64(new[:, 0]), f64(new[:, 1]), f64(k_ft), f64(v_ft), positions,
                                   rot_dim, base, neox, NAME[dtype])
    err = np.abs(f64(out) - ref).max()
    assert err <= TOL[dtype], f"max-abs error {err} > {TOL[dtype]}"
    np.testing.assert_array_equal(bits(v_ft), bits(torch.from_numpy(v2).to(dtype)))
    np.testing.assert_allclose(f64(k_ft), k2, rtol=REL[dtype], atol=ATOL_K[dtype])
    # nothing but the appended positions changed
    k_now, v_now = bits(k_ft), bits(v_ft)
    for b, p in enumerate(positions):
        k_now[b, :, :, p] = k_before[b, :, :, p]
        v_now[b, :, p] = v_before[b, :, p]
    np.testing.assert_array_equal(k_now, k_before)
    np.testing.assert_array_equal(v_now, v_before)


@pytest.mark.parametrize("hq,hkv,d,dtype", FT_GEOMETRIES)
def test_ft_without_rotary_equals_the_standard_layout(device, hq, hkv, d, dtype):
    positions = [3, 0, 700, 64]
    cap = 800
    print(f"ft vs standard {dtype} hq={hq} hkv={hkv} d={d}", flush=True)
    cache, q, new, k_ft, v_ft = ft_case(device, dtype, hq, hkv, d, positions, cap, 31)
    pos = torch.tensor(positions, dtype=torch.int32, device=device)
    out_ft = ops.ft_attend(q, new[:, 0], new[:, 1], k_ft, v_ft, max_position=max(positions), positions=pos)
    out_std = ops.decode_attention(q[:, None], cache, max_seqlen=max(positions) + 1, seqlens=pos,
                                   kv_new=new.contiguous(), kernel="valu")
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(out_ft), bits(out_std[:, 0]))
    k_int, v_int = oracle.ft_layout(bits(cache), ops.ft_pack(dtype))
    np.testing.assert_array_equal(bits(k_ft), k_int)
    np.testing.assert_array_equal(bits(v_ft), v_int)


def test_ft_position_bias_and_positions_agree(device):
    """sequence_len_offset (a uniform bias) and lengths_per_sample (per
    sequence) name the same positions the same way."""
    dtype, hq, hkv, d = torch.float16, 8, 2, 64
    cache, q, new, k1, v1 = ft_case(device, dtype, hq, hkv, d, [41, 41, 41], 64, 41)
    k2, v2 = k1.clone(), v1.clone()
    a = ops.ft_attend(q, new[:, 0], new[:, 1], k1, v1, max_position=41, position_bias=41, rotary_dim=d)
    pos = torch.zeros(3, dtype=torch.int32, device=device) + 40
    b = ops.ft_attend(q, new[:, 0], new[:, 1], k2, v2, max_position=41, positions=pos, position_bias=1,
                      rotary_dim=d)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(a), bits(b))
    np.testing.assert_array_equal(bits(k1), bits(k2))


def test_mha_ft_prefill_then_decode(device):
    """The FT path through the reference-shaped entry points: the prefill
    write of _update_kv_cache (fused_ft_kernel=True) then decode steps of
    _apply_rotary_single_query_attention, first at sequence_len_offset, then
    with lengths_per_sample; the qkv form (kv=None) for MHA."""
    dtype, hq, hkv, d, batch, prompt, cap = torch.bfloat16, 8, 2, 64, 2, 10, 32
    g = torch.Generator(device=device).manual_seed(51)
    params = generation.InferenceParams(max_sequence_len=cap, max_batch_size=batch, fused_ft_kernel=True)
    kv = torch.randn((batch, prompt, 2, hkv, d), generator=g, device=device).to(dtype)
    assert mha._update_kv_cache(kv, params, 0) is kv
    k_cache, v_cache = params.key_value_memory_dict[0]
    assert tuple(k_cache.shape) == (batch, hkv, d // 8, cap, 8) and tuple(v_cache.shape) == (batch, hkv, cap, d)
    ref_k, ref_v = oracle.ft_layout(f64(torch.cat([kv, torch.zeros((batch, cap - prompt, 2, hkv, d), dtype=dtype,
                                                                                 device=device)], 1)), 8)
    positions = [prompt] * batch
    for step in range(3):
        q = torch.randn((batch, 1, hq, d), generator=g, device=device).to(dtype)
        new = torch.randn((batch, 1, 2, hkv, d), generator=g, device=device).to(dtype)
        if step < 2:
            params.sequence_len_offset = positions[0]
        else:
            params.lengths_per_sample = torch.tensor(positions, dtype=torch.int32, device=device)
        out = mha._apply_rotary_single_query_attention(q, params, 0, d, 10000.0, kv=new)
        torch.cuda.synchronize()
        ref, ref_k, ref_v = oracle.ft_decode(f64(q[:, 0]), f64(new[:, 0, 0]), f64(new[:, 0, 1]), ref_k, ref_v,
                                             positions, d, 10000.0, True, "bfloat16")
        assert out.shape == (batch, 1, hq, d)
        err = np.abs(f64(out[:, 0]) - ref).max()
        assert err <= TOL[dtype], f"step {step}: max-abs error {err}"
        positions = [p + 1 for p in positions]
    live = positions[0]
    np.testing.assert_allclose(f64(v_cache)[:, :, :live], ref_v[:, :, :live], rtol=0, atol=0)
    np.testing.assert_allclose(f64(k_cache)[..., :live, :], ref_k[..., :live, :], rtol=REL[dtype],
                               atol=ATOL_K[dtype])
    # the qkv form: q, k, v packed as (B, 1, 3, H, D) for MHA
    params2 = generation.InferenceParams(max_sequence_len=cap, max_batch_size=batch, fused_ft_kernel=True)
    kv2 = torch.randn((batch, prompt, 2, hq, d), generator=g, device=device).to(dtype)
    mha._update_kv_cache(kv2, params2, 3)
    params2.sequence_len_offset = prompt
    qkv = torch.randn((batch, 1, 3, hq, d), generator=g, device=device).to(dtype)
    out = mha._apply_rotary_single_query_attention(qkv, params2, 3, d, 10000.0, rotary_emb_interleaved=True)
    torch.cuda.synchronize()
    k0, v0 = oracle.ft_layout(f64(torch.cat([kv2, torch.zeros((batch, cap - prompt, 2, hq, d), dtype=dtype,
                                                               device=device)], 1)), 8)
    ref, _, _ = oracle.ft_decode(f64(qkv[:, 0, 0]), f64(qkv[:, 0, 1]), f64(qkv[:, 0, 2]), k0, v0,
                                 [prompt] * batch, d, 10000.0, False, "bfloat16")
    assert np.abs(f64(out[:, 0]) - ref).max() <= TOL[dtype]


def test_ft_rejections(device):
    dtype = torch.float16
    cache, q, new, k_ft, v_ft = ft_case(device, dtype, 4, 2, 64, [1, 2], 8, 61)
    with pytest.raises(ValueError):
        ops.ft_attend(q, new[:, 0], new[:, 1], k_ft, v_ft, max_position=8)  # not below capacity
    with pytest.raises(ValueError):
        ops.ft_attend(q, new[:, 0], new[:, 1], k_ft, v_ft, max_position=3, rotary_dim=3)  # odd
    with pytest.raises(ValueError):
        ops.ft_attend(q, new[:, 0], new[:, 1], k_ft, v_ft, max_position=3, rotary_dim=128)  # above head_dim
    with pytest.raises(ValueError):
        ops.ft_attend(q[:, :3], new[:, 0], new[:, 1], k_ft, v_ft, max_position=3)  # heads not a multiple
    with pytest.raises(ValueError):
        ops.ft_attend(q, new[:, 0], new[:, 1], k_ft[:, :, :4], v_ft, max_position=3)  # K/V mismatch
    with pytest.raises(ValueError, match="out shape"):
        ops.ft_attend(q, new[:, 0], new[:, 1], k_ft, v_ft, max_position=3, out=torch.empty_like(q[:1]))
    longer = torch.zeros((2, 9, 2, 2, 64), dtype=dtype, device=device)
    with pytest.raises(ValueError):
        ops.ft_store(longer, k_ft, v_ft)  # more positions than capacity
