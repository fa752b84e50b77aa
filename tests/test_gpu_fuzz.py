"""Seeded random-shape parity sweeps on the GPU: many small configurations
of the pack/unpack round trip, the fused append + attention (both kernels,
forced partitions), attention over host-planned work lists and the FT
decode step, each against the oracle.  The
seeds are fixed, so every run checks the same cases."""
import numpy as np
import pytest
import torch

from hexgen2_amd import ops
from oracle import kv_oracle as oracle

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-3, torch.bfloat16: 8e-3, torch.float32: 2e-5}
INT_VIEW = {torch.float16: torch.int16, torch.bfloat16: torch.int16, torch.float32: torch.int32}
DTYPES = [torch.float16, torch.bfloat16, torch.float32]


def bits(t):
    return t.detach().cpu().contiguous().view(INT_VIEW[t.dtype]).numpy()


def f64(t):
    return t.detach().cpu().double().numpy()


def draw(rng):
    dtype = DTYPES[rng.integers(3)]
    hkv = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([1, 2, 3, 4, 8, 16]))
    d = int(rng.choice([16, 32, 64, 128, 256]))
    batch = int(rng.integers(1, 6))
    lens = [int(x) for x in rng.integers(0, 700, batch)]
    return dtype, hkv, group, d, batch, lens


@pytest.mark.parametrize("seed", range(24))
def test_random_pack_unpack_round_trip(device, seed):
    rng = np.random.default_rng(1000 + seed)
    dtype, hkv, _, d, batch, lens = draw(rng)
    layers, cap = int(rng.integers(1, 5)), max(lens) + int(rng.integers(0, 9))
    print(f"fuzz pack seed={seed} {dtype} L={layers} B={batch} cap={cap} h={hkv} d={d} lens={lens}", flush=True)
    g = torch.Generator(device=device).manual_seed(seed)
    cache = torch.randn((layers, batch, cap, 2, hkv, d), generator=g, device=device).to(dtype)
    packed = ops.pack_live(cache, lens)
    dst = torch.full_like(cache, 3.0)
    ops.unpack_live(packed, dst, lens)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(packed), oracle.pack(list(bits(cache)), lens))
    want = oracle.unpack(oracle.pack(list(bits(cache)), lens), list(bits(torch.full_like(cache, 3.0))), lens)
    np.testing.assert_array_equal(bits(dst), np.stack(want))


@pytest.mark.parametrize("seed", range(32))
def test_random_fused_attention(device, seed):
    rng = np.random.default_rng(2000 + seed)
    dtype, hkv, group, d, batch, lens = draw(rng)
    hq = hkv * group
    kernel = "mfma" if dtype != torch.float32 and d >= 64 and rng.integers(2) else "valu"
    partition = int(rng.choice([0, 64, 128, 320, 512]))
    cap = max(lens) + 2
    print(f"fuzz attend seed={seed} {dtype} B={batch} hq={hq} hkv={hkv} d={d} {kernel} part={partition} "
          f"lens={lens}", flush=True)
    g = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn((batch, 1, hq, d), generator=g, device=device).to(dtype)
    cache = torch.randn((batch, cap, 2, hkv, d), generator=g, device=device).to(dtype)
    kv_new = torch.randn((batch, 2, hkv, d), generator=g, device=device).to(dtype)
    seqlens = torch.tensor(lens, dtype=torch.int32, device=device)
    before = bits(cache)
    out = ops.decode_attention(q, cache, max_seqlen=max(lens) + 1, seqlens=seqlens, kv_new=kv_new,
                               partition=partition, kernel=kernel)
    torch.cuda.synchronize()
    appended = oracle.append(before, bits(kv_new).reshape(batch, -1), lens)
    np.testing.assert_array_equal(bits(cache), appended)
    ref = oracle.attend(f64(q), f64(cache), [n + 1 for n in lens])
    err = np.abs(f64(out) - ref).max()
    assert err <= TOL[dtype], f"max-abs error {err}"


@pytest.mark.parametrize("seed", range(32))
def test_random_work_list_attention(device, seed):
    """Attention over host-planned work lists (hexkv_attend_plan) on random
    shapes: chunk sizes from 64 positions to beyond the grid's 4096 cap,
    a length bias, with and without the fused append (empty rows then give
    zero outputs)."""
    rng = np.random.default_rng(4000 + seed)
    dtype, hkv, group, d, batch, lens = draw(rng)
    hq = hkv * group
    kernel = "mfma" if dtype != torch.float32 and d >= 64 and rng.integers(2) else "valu"
    partition = int(rng.choice([0, 64, 128, 320, 512, 4160]))
    fused = bool(rng.integers(2))
    bias = int(rng.integers(0, 4))
    if seed % 4 == 0:  # an empty row: no append, no bias
        fused, bias, lens[0] = False, 0, 0
    extra = 1 if fused else 0
    attended = [n + bias + extra for n in lens]
    cap = max(lens) + bias + 2
    print(f"fuzz list seed={seed} {dtype} B={batch} hq={hq} hkv={hkv} d={d} {kernel} part={partition} "
          f"fused={fused} bias={bias} lens={lens}", flush=True)
    g = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn((batch, 1, hq, d), generator=g, device=device).to(dtype)
    cache = torch.randn((batch, cap, 2, hkv, d), generator=g, device=device).to(dtype)
    kv_new = torch.randn((batch, 2, hkv, d), generator=g, device=device).to(dtype) if fused else None
    seqlens = torch.tensor(lens, dtype=torch.int32, device=device)
    before = bits(cache)
    out = torch.full_like(q, 7.0)
    ops.decode_attention(q, cache, max_seqlen=max(attended), seqlens=seqlens, seqlen_bias=bias,
                         kv_new=kv_new, out=out, partition=partition, kernel=kernel, lens=lens)
    torch.cuda.synchronize()
    if fused:
        appended = oracle.append(before, bits(kv_new).reshape(batch, -1), [n + bias for n in lens])
        np.testing.assert_array_equal(bits(cache), appended)
    else:
        np.testing.assert_array_equal(bits(cache), before)
    got = f64(out)
    live = [b for b in range(batch) if attended[b] > 0]
    for b in range(batch):
        if attended[b] == 0:
            assert not got[b].any(), f"empty row {b} not zero"
    if live:
        ref = oracle.attend(f64(q)[live], f64(cache)[live], [attended[b] for b in live])
        err = np.abs(got[live] - ref).max()
        assert err <= TOL[dtype], f"max-abs error {err}"


@pytest.mark.parametrize("seed", range(16))
def test_random_ft_decode(device, seed):
    rng = np.random.default_rng(3000 + seed)
    dtype, hkv, group, d, batch, lens = draw(rng)
    hq = hkv * group
    cap = max(lens) + 2
    rot = int(rng.choice([0, d // 2, d]))
    neox = bool(rng.integers(2))
    print(f"fuzz ft seed={seed} {dtype} B={batch} hq={hq} hkv={hkv} d={d} rot={rot} neox={neox} lens={lens}",
          flush=True)
    g = torch.Generator(device=device).manual_seed(seed)
    cache = torch.randn((batch, cap, 2, hkv, d), generator=g, device=device).to(dtype)
    q = torch.randn((batch, hq, d), generator=g, device=device).to(dtype)
    new = torch.randn((batch, 2, hkv, d), generator=g, device=device).to(dtype)
    pack = ops.ft_pack(dtype)
    k_int, v_int = oracle.ft_layout(bits(cache), pack)
    k_ft = torch.from_numpy(k_int).view(dtype).to(device)
    v_ft = torch.from_numpy(v_int).view(dtype).to(device)
    pos = torch.tensor(lens, dtype=torch.int32, device=device)
    out = ops.ft_attend(q, new[:, 0], new[:, 1], k_ft, v_ft, max_position=max(lens), positions=pos,
                        rotary_dim=rot, rotary_neox=neox)
    torch.cuda.synchronize()
    name = {torch.float16: "float16", torch.bfloat16: "bfloat16", torch.float32: "float32"}[dtype]
    ref, _, v2 = oracle.ft_decode(f64(q), f64(new[:, 0]), f64(new[:, 1]), f64(k_ft), f64(v_ft), lens, rot,
                                  10000.0, neox, name)
    err = np.abs(f64(out) - ref).max()
    assert err <= TOL[dtype], f"max-abs error {err}"
    np.testing.assert_array_equal(bits(v_ft), bits(torch.from_numpy(v2).to(dtype)))
