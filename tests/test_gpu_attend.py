"""GPU parity of decode attention (hexkv_attend) against the float64 oracle.

Tolerances (max-abs, inputs rounded to the dtype first, oracle in float64):
fp16 2e-3, bf16 8e-3, fp32 2e-5.  The fused append must also write the new
row bit-exactly and touch nothing else.  Both score kernels are checked: the
VALU kernel (every dtype and head_dim) and the MFMA kernel (16-bit,
head_dim >= 64).
"""
import ctypes

import numpy as np
import pytest
import torch

from hexgen2_amd import _lib, ops
from oracle import kv_oracle as oracle

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-3, torch.bfloat16: 8e-3, torch.float32: 2e-5}
INT_VIEW = {torch.float16: torch.int16, torch.bfloat16: torch.int16, torch.float32: torch.int32}


def bits(t):
    return t.detach().cpu().contiguous().view(INT_VIEW[t.dtype]).numpy()


def f64(t):
    return t.detach().cpu().double().numpy()


def make(batch, cap, hq, hkv, d, dtype, seed, device, q_len=1):
    g = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn((batch, q_len, hq, d), generator=g, device=device).to(dtype)
    cache = torch.randn((batch, cap, 2, hkv, d), generator=g, device=device).to(dtype)
    return q, cache


def check(out, q, cache, lens, dtype, causal=False, scale=None):
    ref = oracle.attend(f64(q), f64(cache), lens, causal=causal, softmax_scale=scale)
    err = np.abs(f64(out) - ref).max()
    assert err <= TOL[dtype], f"max-abs error {err} > {TOL[dtype]}"
    return err


# (hq, hkv, d, dtype): the geometry of every configuration plus edge groups
GEOMETRIES = [
    (4, 4, 16, torch.float32),     # tiny llama, fp32
    (4, 2, 32, torch.float16),     # reference fixture
    (32, 4, 64, torch.float16),    # TinyLlama-1.1B
    (32, 32, 128, torch.float16),  # Llama-2-7B
    (8, 1, 128, torch.bfloat16),   # Llama-2-70B TP-8 share
    (32, 8, 128, torch.bfloat16),  # Llama-3-8B
    (32, 2, 128, torch.bfloat16),  # group 16 -> two head groups per KV head
    (6, 2, 64, torch.float16),     # group 3 -> one head per workgroup
    (4, 2, 256, torch.bfloat16),   # head_dim 256
    (8, 8, 128, torch.float32),    # fp32, 32 lanes per position
]


def kernels_for(dtype, d):
    return ["valu", "mfma"] if dtype != torch.float32 and d >= 64 else ["valu"]


CASES = [(hq, hkv, d, dtype, kernel) for hq, hkv, d, dtype in GEOMETRIES for kernel in kernels_for(dtype, d)]


@pytest.mark.parametrize("hq,hkv,d,dtype,kernel", CASES)
def test_ragged_lengths_within_tolerance(device, hq, hkv, d, dtype, kernel):
    lens = [1, 15, 16, 17, 63, 64, 65, 700, 1500, 2049]
    cap = 2112
    print(f"attend {kernel} hq={hq} hkv={hkv} d={d} {dtype} lens={lens}", flush=True)
    q, cache = make(len(lens), cap, hq, hkv, d, dtype, 1, device)
    seqlens = torch.tensor(lens, dtype=torch.int32, device=device)
    for partition in (0, 64, 192, 512):
        out = ops.decode_attention(q, cache, max_seqlen=max(lens), seqlens=seqlens, partition=partition,
                                   kernel=kernel)
        torch.cuda.synchronize()
        check(out, q, cache, lens, dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_uniform_length_and_scale(device, dtype):
    q, cache = make(3, 300, 16, 4, 128, dtype, 2, device)
    for kernel in kernels_for(dtype, 128):
        out = ops.decode_attention(q, cache, max_seqlen=257, seqlen_bias=257, softmax_scale=0.05, kernel=kernel)
        check(out, q, cache, [257] * 3, dtype, scale=0.05)


@pytest.mark.parametrize("kernel", ["valu", "mfma"])
def test_large_scores_rescale_running_max(device, kernel):
    # scores growing along the sequence force repeated rescales of the
    # running maximum; a large scale makes them span hundreds of log2 units
    q, cache = make(2, 600, 8, 2, 128, torch.bfloat16, 13, device)
    ramp = torch.linspace(0.1, 4.0, 600, device=device)[None, :, None, None]
    cache[:, :, 0] = (cache[:, :, 0].float() * ramp).to(torch.bfloat16)
    out = ops.decode_attention(q, cache, max_seqlen=600, seqlen_bias=600, softmax_scale=0.5, kernel=kernel)
    check(out, q, cache, [600, 600], torch.bfloat16, scale=0.5)


def test_single_key_returns_value_exactly(device):
    q, cache = make(2, 8, 8, 2, 64, torch.bfloat16, 3, device)
    out = ops.decode_attention(q, cache, max_seqlen=1, seqlen_bias=1)
    want = cache[:, 0, 1].repeat_interleave(4, dim=1)
    assert torch.equal(out[:, 0], want)


def test_dominant_key_selects_value(device):
    q, cache = make(1, 40, 4, 4, 128, torch.float16, 4, device)
    q.zero_()
    q[0, 0, :, 0] = 1.0
    cache[0, :, 0].zero_()
    cache[0, 17, 0, :, 0] = 60.0
    out = ops.decode_attention(q, cache, max_seqlen=40, seqlen_bias=40, softmax_scale=1.0)
    torch.testing.assert_close(out[0, 0], cache[0, 17, 1], rtol=0, atol=1e-3)


def test_zero_length_rows_give_zeros(device):
    q, cache = make(3, 16, 8, 2, 64, torch.float16, 5, device)
    lens = torch.tensor([0, 5, 0], dtype=torch.int32, device=device)
    out = torch.full_like(q, 9.0)  # stale values must be overwritten
    ops.decode_attention(q, cache, max_seqlen=5, seqlens=lens, out=out)
    assert (out[0] == 0).all() and (out[2] == 0).all()
    check(out[1:2], q[1:2], cache[1:2], [5], torch.float16)
    out = torch.full_like(q, 9.0)
    ops.decode_attention(q, cache, max_seqlen=5, seqlens=torch.zeros(3, dtype=torch.int32, device=device), out=out)
    assert (out == 0).all()


FUSED = [(32, 8, 128, torch.bfloat16, "valu"), (32, 8, 128, torch.bfloat16, "mfma"),
         (32, 4, 64, torch.float16, "valu"), (32, 4, 64, torch.float16, "mfma"),
         (4, 4, 16, torch.float32, "valu"), (32, 2, 128, torch.bfloat16, "mfma"),
         (8, 1, 256, torch.bfloat16, "mfma"), (8, 1, 256, torch.bfloat16, "valu")]


@pytest.mark.parametrize("hq,hkv,d,dtype,kernel", FUSED)
def test_fused_append_writes_row_and_attends_it(device, hq, hkv, d, dtype, kernel):
    lens = [0, 5, 15, 16, 63, 64, 1023, 1024, 3000]
    cap = 3100
    print(f"fused {kernel} hq={hq} hkv={hkv} d={d} {dtype}", flush=True)
    q, cache = make(len(lens), cap, hq, hkv, d, dtype, 6, device)
    g = torch.Generator(device=device).manual_seed(7)
    kv_new = torch.randn((len(lens), 2, hkv, d), generator=g, device=device).to(dtype)
    before = bits(cache)
    seqlens = torch.tensor(lens, dtype=torch.int32, device=device)
    out = ops.decode_attention(q, cache, max_seqlen=max(lens) + 1, seqlens=seqlens, kv_new=kv_new, kernel=kernel)
    torch.cuda.synchronize()
    want_cache = oracle.append(before, bits(kv_new), lens)
    np.testing.assert_array_equal(bits(cache), want_cache)
    check(out, q, cache, [n + 1 for n in lens], dtype)


@pytest.mark.parametrize("kernel", ["valu", "mfma"])
def test_fused_append_with_bias_matches_unfused(device, kernel):
    q, cache = make(4, 200, 32, 8, 128, torch.bfloat16, 8, device)
    kv_new = torch.randn((4, 2, 8, 128), device=device).to(torch.bfloat16)
    base = torch.tensor([10, 0, 150, 98], dtype=torch.int32, device=device)
    c1, c2 = cache.clone(), cache.clone()
    o1 = ops.decode_attention(q, c1, max_seqlen=156, seqlens=base, seqlen_bias=5, kv_new=kv_new, kernel=kernel)
    ops.append_kv(c2, kv_new.reshape(4, -1), base, position_bias=5)
    o2 = ops.decode_attention(q, c2, max_seqlen=156, seqlens=base, seqlen_bias=6, kernel=kernel)
    assert torch.equal(c1, c2)
    # the same keys in the same order; only the summation grouping may differ
    torch.testing.assert_close(o1, o2, rtol=0, atol=8e-3)
    check(o1, q, c2, [n + 6 for n in [10, 0, 150, 98]], torch.bfloat16)


@pytest.mark.parametrize("dtype,d,kernel", [(torch.float32, 32, "valu"), (torch.float16, 32, "valu"),
                                            (torch.float16, 64, "mfma"), (torch.bfloat16, 128, "mfma")])
def test_causal_prefill_rows(device, dtype, d, kernel):
    q, cache = make(2, 40, 4, 2, d, dtype, 9, device, q_len=7)
    out = ops.decode_attention(q, cache, max_seqlen=40, seqlen_bias=7, causal=True, kernel=kernel)
    check(out, q, cache, [7, 7], dtype, causal=True)
    seqlens = torch.tensor([30, 7], dtype=torch.int32, device=device)
    out = ops.decode_attention(q, cache, max_seqlen=40, seqlens=seqlens, causal=True, kernel=kernel)
    check(out, q, cache, [30, 7], dtype, causal=True)


@pytest.mark.parametrize("kernel", ["valu", "mfma"])
def test_strided_cache_view_batch_offset(device, kernel):
    # the view _update_kv_cache returns: cache[b0:b1, :offset+1]
    q, cache = make(5, 64, 8, 2, 64, torch.float16, 10, device)
    view = cache[1:4, :33]
    out = ops.decode_attention(q[1:4], view, max_seqlen=33, seqlen_bias=33, kernel=kernel)
    check(out, q[1:4], view, [33] * 3, torch.float16)


@pytest.mark.parametrize("kernel", ["valu", "mfma"])
def test_repeatable(device, kernel):
    q, cache = make(8, 4096, 32, 8, 128, torch.bfloat16, 11, device)
    lens = torch.randint(1, 4096, (8,), dtype=torch.int32, device=device)
    a = ops.decode_attention(q, cache, max_seqlen=4096, seqlens=lens, kernel=kernel)
    b = ops.decode_attention(q, cache, max_seqlen=4096, seqlens=lens, kernel=kernel)
    assert torch.equal(a, b)


def test_valu_and_mfma_agree(device):
    q, cache = make(6, 3000, 32, 8, 128, torch.bfloat16, 14, device)
    lens = torch.tensor([1, 17, 300, 1025, 2999, 2048], dtype=torch.int32, device=device)
    a = ops.decode_attention(q, cache, max_seqlen=3000, seqlens=lens, kernel="valu")
    b = ops.decode_attention(q, cache, max_seqlen=3000, seqlens=lens, kernel="mfma")
    torch.testing.assert_close(a.float(), b.float(), rtol=0, atol=8e-3)


@pytest.mark.parametrize("kernel", ["valu", "mfma"])
def test_many_ragged_rows(device, kernel):
    # 300 rows of lengths 0..4000 (every 7th empty, one long): partitions of
    # very different counts per row, most rows inside one partition
    g = torch.Generator().manual_seed(15)
    lens = torch.randint(0, 600, (300,), generator=g)
    lens[::7] = 0
    lens[5] = 4000
    q, cache = make(300, 4001, 16, 2, 64, torch.float16, 15, device)
    seqlens = lens.to(torch.int32).to(device)
    live = [i for i, n in enumerate(lens.tolist()) if n > 0]
    empty = [i for i, n in enumerate(lens.tolist()) if n == 0]
    ref = oracle.attend(f64(q)[live], f64(cache)[live], [int(lens[i]) for i in live])
    for partition in (0, 256):
        out = ops.decode_attention(q, cache, max_seqlen=4000, seqlens=seqlens, kernel=kernel, partition=partition)
        assert np.abs(f64(out)[live] - ref).max() <= TOL[torch.float16], partition
        assert (out[empty] == 0).all(), partition


def test_validation_errors(device):
    q, cache = make(2, 16, 8, 2, 64, torch.float16, 12, device)
    with pytest.raises(ValueError):
        ops.decode_attention(q, cache, max_seqlen=17, seqlen_bias=17)  # beyond capacity
    with pytest.raises(NotImplementedError):
        qq, cc = make(1, 8, 2, 1, 48, torch.float16, 0, device)
        ops.decode_attention(qq, cc, max_seqlen=4, seqlen_bias=4)  # head_dim 48 not compiled
    with pytest.raises(ValueError):
        ops.decode_attention(q.float(), cache, max_seqlen=4, seqlen_bias=4)  # dtype mismatch
    with pytest.raises(NotImplementedError):
        qq, cc = make(1, 8, 2, 1, 32, torch.float16, 0, device)
        ops.decode_attention(qq, cc, max_seqlen=4, seqlen_bias=4, kernel="mfma")  # head_dim < 64
    with pytest.raises(NotImplementedError):
        qq, cc = make(1, 8, 2, 1, 64, torch.float32, 0, device)
        ops.decode_attention(qq, cc, max_seqlen=4, seqlen_bias=4, kernel="mfma")  # fp32
    with pytest.raises(ValueError):
        ops.decode_attention(q, cache, max_seqlen=4, seqlen_bias=4, softmax_scale=-1.0)
    # an output smaller than q is refused on the host, before the kernel could write past it
    with pytest.raises(ValueError, match="out shape"):
        ops.decode_attention(q, cache, max_seqlen=4, seqlen_bias=4, out=torch.empty_like(q[:1]))
    with pytest.raises(ValueError, match="out shape"):
        ops.decode_attention_noalloc(q, cache, torch.empty_like(q[:, :, :4]), max_seqlen=4, seqlen_bias=4)


# ------------------------------------------------------------- work lists ---
# hexkv_attend_plan's list (compact, largest items first, lengths carried by
# the items) against the oracle: every geometry, both kernels, the library's
# chunk choice and forced chunks, with and without the fused append.

@pytest.mark.parametrize("hq,hkv,d,dtype,kernel", CASES)
def test_work_list_ragged_within_tolerance(device, hq, hkv, d, dtype, kernel):
    lens = [0, 1, 15, 16, 17, 63, 64, 65, 700, 1500, 2047, 2048]
    cap = 2112
    print(f"work list {kernel} hq={hq} hkv={hkv} d={d} {dtype}", flush=True)
    q, cache = make(len(lens), cap, hq, hkv, d, dtype, 41, device)
    g = torch.Generator(device=device).manual_seed(42)
    kv_new = torch.randn((len(lens), 2, hkv, d), generator=g, device=device).to(dtype)
    seqlens = torch.tensor(lens, dtype=torch.int32, device=device)
    before = bits(cache)
    want_cache = oracle.append(before, bits(kv_new), lens)
    for partition in (0, 64, 384, 1024):
        c = cache.clone()
        out = ops.decode_attention(q, c, max_seqlen=max(lens) + 1, seqlens=seqlens, kv_new=kv_new,
                                   partition=partition, kernel=kernel, lens=lens)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(c), want_cache)
        check(out, q, c, [n + 1 for n in lens], dtype)
    # without the append: the empty row gives zeros
    out = torch.full_like(q, 9.0)
    ops.decode_attention(q, cache, max_seqlen=max(lens), seqlens=seqlens, kernel=kernel, lens=lens, out=out)
    assert (out[0] == 0).all()
    check(out[1:], q[1:], cache[1:], lens[1:], dtype)


@pytest.mark.parametrize("hq,hkv,d,dtype,kernel", [(32, 4, 64, torch.float16, "mfma"),
                                                   (32, 32, 128, torch.float16, "valu"),
                                                   (8, 1, 128, torch.bfloat16, "mfma"),
                                                   (4, 4, 16, torch.float32, "valu")])
def test_output_at_odd_element_offset(device, hq, hkv, d, dtype, kernel):
    """Output rows one element past a 16-byte boundary (a view into a larger
    buffer): the kernels store four outputs at once only where the address
    allows it, element by element otherwise.  The values must equal those
    written to an aligned output bit for bit -- on the grid, on a work list
    merged inside the attention kernel and on one merged by a second launch
    -- and the element before the view stays untouched."""
    lens = [0, 5, 64, 700, 2047]
    q, cache = make(len(lens), 2112, hq, hkv, d, dtype, 17, device)
    seqlens = torch.tensor(lens, dtype=torch.int32, device=device)
    for mode in ("grid", "list", "two-launch"):
        print(f"odd output offset {kernel} hq={hq} hkv={hkv} d={d} {dtype} {mode}", flush=True)
        kw = {} if mode == "grid" else dict(lens=lens, single_launch=mode == "list")
        aligned = ops.decode_attention(q, cache, max_seqlen=max(lens), seqlens=seqlens, partition=64,
                                       kernel=kernel, **kw)
        buf = torch.full((q.numel() + 1,), 5.0, dtype=dtype, device=device)
        odd = buf[1:].view(q.shape)
        assert odd.data_ptr() % 16 != 0
        ops.decode_attention(q, cache, max_seqlen=max(lens), seqlens=seqlens, partition=64, kernel=kernel,
                             out=odd, **kw)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(odd), bits(aligned))
        assert buf[0].item() == 5.0
        assert (aligned[0] == 0).all()
        check(aligned[1:], q[1:], cache[1:], lens[1:], dtype)


# (hq, hkv, dtype): geometries of the row-block kernel (head_dim 128): items
# of 2 adjacent KV heads for grouped queries, 8 (or 4) for one query head
# per KV head
ROWS_GEOMETRIES = [
    (32, 8, torch.bfloat16),   # Llama-3-8B
    (32, 8, torch.float16),
    (32, 32, torch.float16),   # Llama-2-7B: 8 KV heads per item
    (16, 8, torch.bfloat16),   # group 2
    (8, 4, torch.bfloat16),    # group 2, 2 blocks per row
    (4, 4, torch.float16),     # group 1, 4 KV heads: one block of 4
    (8, 2, torch.bfloat16),    # group 4, one block of 2 per row
    (6, 6, torch.float16),     # group 1, 6 KV heads: three blocks of 2
]


@pytest.mark.parametrize("hq,hkv,dtype", ROWS_GEOMETRIES)
def test_row_block_kernel_ragged_within_tolerance(device, hq, hkv, dtype):
    """The row-block kernel over ragged lists (empty rows, single keys,
    rows ending on and around chunk boundaries, up to 64 pieces per row
    merged in the kernel): within tolerance of the oracle, the fused append
    bit-exact, and the device status clear."""
    lens = [0, 1, 15, 16, 17, 63, 64, 65, 700, 1500, 2047, 2048]
    cap = 2112
    print(f"row-block hq={hq} hkv={hkv} {dtype}", flush=True)
    q, cache = make(len(lens), cap, hq, hkv, 128, dtype, 43, device)
    g = torch.Generator(device=device).manual_seed(44)
    kv_new = torch.randn((len(lens), 2, hkv, 128), generator=g, device=device).to(dtype)
    seqlens = torch.tensor(lens, dtype=torch.int32, device=device)
    want_cache = oracle.append(bits(cache), bits(kv_new), lens)
    ops.device_status()
    for partition in (0, 48, 144, 512):
        c = cache.clone()
        out = ops.decode_attention(q, c, max_seqlen=max(lens) + 1, seqlens=seqlens, kv_new=kv_new,
                                   partition=partition, kernel="rows", lens=lens)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(c), want_cache)
        check(out, q, c, [n + 1 for n in lens], dtype)
    out = torch.full_like(q, 9.0)
    ops.decode_attention(q, cache, max_seqlen=max(lens), seqlens=seqlens, kernel="rows", lens=lens, out=out)
    assert (out[0] == 0).all()
    check(out[1:], q[1:], cache[1:], lens[1:], dtype)
    assert ops.device_status() & _lib.STATUS_ERRORS == 0


@pytest.mark.parametrize("hq,hkv,dtype", ROWS_GEOMETRIES[:3])
def test_row_block_kernel_agrees_with_head_items(device, hq, hkv, dtype):
    """Row-block and one-head-per-item lists of the same call: outputs within
    the bf16/fp16 tolerance of each other, caches bit-identical."""
    lens = [300, 5, 1200, 77, 2500, 640, 0, 4095]
    q, cache = make(len(lens), 4160, hq, hkv, 128, dtype, 45, device)
    g = torch.Generator(device=device).manual_seed(46)
    kv_new = torch.randn((len(lens), 2, hkv, 128), generator=g, device=device).to(dtype)
    seqlens = torch.tensor(lens, dtype=torch.int32, device=device)
    c_rows, c_head = cache.clone(), cache.clone()
    o_rows = ops.decode_attention(q, c_rows, max_seqlen=max(lens) + 1, seqlens=seqlens, kv_new=kv_new,
                                  kernel="rows", lens=lens)
    o_head = ops.decode_attention(q, c_head, max_seqlen=max(lens) + 1, seqlens=seqlens, kv_new=kv_new,
                                  kernel="valu", lens=lens)
    torch.cuda.synchronize()
    assert torch.equal(c_rows.view(torch.int16), c_head.view(torch.int16))
    torch.testing.assert_close(o_rows.float(), o_head.float(), rtol=0, atol=TOL[dtype])


@pytest.mark.parametrize("kernel", ["valu", "mfma", "rows"])
def test_work_list_same_on_every_stream(device, kernel):
    """Workgroups reach the XCDs round-robin from a start XCD that depends on
    the hardware queue; the kernels run each XCD's share of a list on that
    XCD whatever the start.  The same fused call on four streams (the queues
    of one process start at different XCDs): outputs and caches bit-identical,
    within tolerance of the oracle, no error flag (the placement flag among
    them)."""
    lens = [3000, 17, 1200, 640, 2047, 95, 4000, 333]
    q, cache = make(len(lens), 4160, 32, 8, 128, torch.bfloat16, 48, device)
    g = torch.Generator(device=device).manual_seed(49)
    kv_new = torch.randn((len(lens), 2, 8, 128), generator=g, device=device).to(torch.bfloat16)
    seqlens = torch.tensor(lens, dtype=torch.int32, device=device)
    streams = [torch.cuda.current_stream()] + [torch.cuda.Stream() for _ in range(3)]
    ops.device_status()
    results = []
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(st):
            c = cache.clone()
            out = ops.decode_attention(q, c, max_seqlen=max(lens) + 1, seqlens=seqlens, kv_new=kv_new,
                                       kernel=kernel, lens=lens)
        torch.cuda.synchronize()
        results.append((out, c))
    for out, c in results[1:]:
        assert torch.equal(out, results[0][0])
        assert torch.equal(c.view(torch.int16), results[0][1].view(torch.int16))
    check(results[0][0], q, results[0][1], [n + 1 for n in lens], torch.bfloat16)
    assert ops.device_status() & _lib.STATUS_ERRORS == 0


def test_list_planned_for_other_xcd_count_is_refused(device):
    """A split list dealt over another XCD count than the device's would put
    a segment's items on two XCDs, where the in-kernel merge reads stale
    partials: hexkv_attend refuses it before launching."""
    lib = _lib.load()
    lens = [900, 3000, 40]
    q, cache = make(len(lens), 3100, 32, 8, 128, torch.bfloat16, 50, device)
    out = torch.full_like(q, 3.0)
    seqlens = torch.tensor(lens, dtype=torch.int32, device=device)
    xcds = ops.device_xcds(0)
    p = ops._attend_params(q, cache, out, seqlens, 0, max(lens), None, False, None, 128, "valu")
    p.work_xcds = 4 if xcds != 4 else 2
    c_lens = (ctypes.c_int32 * len(lens))(*lens)
    n, mp = ctypes.c_int32(), ctypes.c_int32()
    _lib.check(lib.hexkv_attend_plan(ctypes.byref(p), c_lens, None, 0, None, 0, ctypes.byref(n), ctypes.byref(mp)),
               "plan")
    items = torch.empty((n.value, 8), dtype=torch.int32)
    parts = torch.empty(len(lens) * 32, dtype=torch.int32)
    _lib.check(lib.hexkv_attend_plan(ctypes.byref(p), c_lens, ctypes.c_void_p(items.data_ptr()), n.value,
                                     ctypes.c_void_p(parts.data_ptr()), parts.numel(), ctypes.byref(n),
                                     ctypes.byref(mp)), "plan")
    assert mp.value > 1  # split rows: the in-kernel merge would run
    items_d, parts_d = items.to(device), parts.to(device)
    p.work_items_dev, p.work_parts_dev = items_d.data_ptr(), parts_d.data_ptr()
    p.n_work_items, p.work_max_parts = n.value, mp.value
    need = int(lib.hexkv_attend_workspace_bytes(ctypes.byref(p)))
    ws = torch.zeros(need, dtype=torch.uint8, device=device)
    rc = lib.hexkv_attend(ctypes.byref(p), ctypes.c_void_p(ws.data_ptr()), need,
                          ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == _lib.HEXKV_EINVAL and b"XCDs" in lib.hexkv_last_error()
    torch.cuda.synchronize()
    assert (out == 3.0).all(), "nothing was launched"


def test_list_planned_for_another_kernel_is_skipped_and_reported(device):
    """A row-block list launched as the one-head-per-item kernel (head groups
    of another size): every item is skipped, nothing is written, and the
    status word says so (check_device_status raises)."""
    lens = [100, 900, 33]
    q, cache = make(len(lens), 1024, 32, 8, 128, torch.bfloat16, 47, device)
    seqlens = torch.tensor(lens, dtype=torch.int32, device=device)
    out = torch.full_like(q, 7.0)
    plan = ops.AttendPlan(q, cache, out, max_seqlens=[max(lens)], seqlens=seqlens, kernel="rows")
    work = ops._plan_work(plan.params, lens, device)
    assert work.kernel == _lib.KERNELS["rows"]
    plan.fix_work_list(work)
    plan.params.kernel = _lib.KERNELS["valu"]  # launch it as another kernel
    ops.device_status()
    plan(q, cache, out, None, 0, max(lens))
    torch.cuda.synchronize()
    assert (out == 7.0).all(), "a skipped item wrote"
    with pytest.raises(ValueError, match="another attention kernel"):
        ops.check_device_status()
    assert ops.device_status() == 0  # the check cleared it
    plan.params.kernel = work.kernel  # as planned: every output written
    plan(q, cache, out, None, 0, max(lens))
    check(out, q, cache, lens, torch.bfloat16)
    assert ops.device_status() & _lib.STATUS_ERRORS == 0


@pytest.mark.parametrize("kernel", ["valu", "mfma"])
def test_attend_plan_work_list_matches_grid_over_steps(device, kernel):
    # AttendPlan with host lengths (a list per step, shared by the layers)
    # against the same plan over the device lengths only (uniform grid)
    lens = [300, 5, 1200, 77, 2500, 640]
    L, steps = 3, 4
    cap = max(lens) + steps
    g = torch.Generator(device=device).manual_seed(43)
    q = torch.randn((L, len(lens), 1, 32, 128), generator=g, device=device).to(torch.bfloat16)
    kv = torch.randn((L, len(lens), 2, 8, 128), generator=g, device=device).to(torch.bfloat16)
    caches = torch.randn((L, len(lens), cap, 2, 8, 128), generator=g, device=device).to(torch.bfloat16)
    c_list, c_grid = caches.clone(), caches.clone()
    seqlens = torch.tensor(lens, dtype=torch.int32, device=device)
    o_list, o_grid = torch.empty_like(q[0]), torch.empty_like(q[0])
    maxes = [max(lens) + t + 1 for t in range(steps)]
    p_list = ops.AttendPlan(q[0], c_list[0], o_list, max_seqlens=maxes, seqlens=seqlens, kv_new=kv[0],
                            kernel=kernel, lens=lens)
    p_grid = ops.AttendPlan(q[0], c_grid[0], o_grid, max_seqlens=maxes, seqlens=seqlens, kv_new=kv[0],
                            kernel=kernel)
    for t in range(steps):
        for l in range(L):
            p_list(q[l], c_list[l], o_list, kv[l], t, maxes[t])
            p_grid(q[l], c_grid[l], o_grid, kv[l], t, maxes[t])
            torch.cuda.synchronize()
            torch.testing.assert_close(o_list.float(), o_grid.float(), rtol=0, atol=8e-3)
            check(o_list, q[l], c_list[l], [n + t + 1 for n in lens], torch.bfloat16)
    assert torch.equal(c_list.view(torch.int16), c_grid.view(torch.int16))


@pytest.mark.parametrize("hq,hkv,d,dtype,kernel", [(8, 1, 128, torch.bfloat16, "mfma"),
                                                   (32, 8, 128, torch.bfloat16, "valu"),
                                                   (32, 4, 64, torch.float16, "valu"),
                                                   (4, 2, 256, torch.bfloat16, "valu")])
def test_rows_with_hundreds_of_partitions(device, hq, hkv, d, dtype, kernel):
    """A 20,000-position row cut into 64-position partitions has 313 of them:
    the merge kernel stages their weights through LDS 256 at a time (the
    path beyond its register fast path).  Grid and work list, with short
    and empty rows beside it, against the float64 oracle."""
    lens = [20000, 3, 0, 700]
    cap = 20032
    q, cache = make(len(lens), cap, hq, hkv, d, dtype, 9, device)
    # queries at three times the keys' scale: a row's weight then sits on few
    # keys, so a merge stage dropped or weighted wrongly moves the output far
    # past the tolerance (at unit scale 20,000 keys average it away)
    q = (3 * q.float()).to(dtype)
    seqlens = torch.tensor(lens, dtype=torch.int32, device=device)
    print(f"attend {kernel} hq={hq} hkv={hkv} d={d} {dtype}: 313 partitions", flush=True)
    live = [b for b, n in enumerate(lens) if n]
    ref = oracle.attend(f64(q)[live], f64(cache)[live], [lens[b] for b in live])
    for listed in (False, True):
        out = ops.decode_attention(q, cache, max_seqlen=max(lens), seqlens=seqlens, partition=64, kernel=kernel,
                                   lens=lens if listed else None)
        torch.cuda.synchronize()
        # absolute error up to 1, relative above (16-bit rounding grows with the output)
        err = (np.abs(f64(out)[live] - ref) / np.maximum(1.0, np.abs(ref))).max()
        assert err <= TOL[dtype], f"{'work list' if listed else 'grid'}: max-abs {err}"
        assert (out[2] == 0).all(), "empty row not zero"
