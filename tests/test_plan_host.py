"""Host-side checks (no GPU) of the decode-attention planning code.

* AttendPlan's per-call geometry comparison: an AttendPlan patches only
  addresses into a parameter block built once, so a call with a tensor of
  another shape, stride, dtype or device, or a short or non-contiguous
  kv_new, must raise ValueError before anything is launched.  The comparison
  is a pure function of tensor metadata, exercised here on CPU tensors.
* hexkv_attend_plan (host code of the C library): the work list covers
  every attended position of every (row, head group) exactly once, the
  partition numbers and counts agree with the merge's view, the order is
  empty rows, full chunks, then the shorter last chunks from the longest
  down, and the library's chunk choice follows its three regimes; planned
  for the device's XCDs, every item of a split (row, head group) sits at one
  index modulo the XCD count, with the same order within each XCD.
"""
import ctypes

import numpy as np
import pytest
import torch

from hexgen2_amd import _lib, ops


def tensors(dtype=torch.bfloat16):
    q = torch.zeros((4, 1, 32, 128), dtype=dtype)
    cache = torch.zeros((4, 64, 2, 8, 128), dtype=dtype)
    out = torch.zeros((4, 1, 32, 128), dtype=dtype)
    kv_new = torch.zeros((4, 2, 8, 128), dtype=dtype)
    return q, cache, out, kv_new


def check(built, called):
    ops._check_plan_geometry(ops._plan_geometry(*built), ops._plan_geometry(*called))


def test_same_geometry_passes():
    a, b = tensors(), tensors()
    check(a, b)
    # other addresses, same layout: still the same geometry
    big = torch.zeros((2, 4, 64, 2, 8, 128), dtype=torch.bfloat16)
    q, _, out, kv = tensors()
    check((q, big[0], out, kv), (q, big[1], out, kv))


@pytest.mark.parametrize("which,bad", [
    ("q", lambda q: torch.zeros((4, 1, 64, 128), dtype=q.dtype)[:, :, :32]),  # same shape, other strides
    ("out", lambda o: torch.zeros((4, 2, 32, 128), dtype=o.dtype)[:, :1]),  # row stride 2x
    ("cache", lambda c: c.to(torch.float16)),                               # 16-bit of another kind
    ("cache", lambda c: torch.zeros((4, 65, 2, 8, 128), dtype=c.dtype)[:, :64]),  # other batch stride
    ("kv_new", lambda k: k[:3]),                                            # short
    ("kv_new", lambda k: torch.zeros((2, 4, 8, 128), dtype=k.dtype).transpose(0, 1)),  # not contiguous
    ("kv_new", lambda k: k.to("meta")),                                     # other device
    ("kv_new", lambda k: None),                                             # fused plan, no kv_new
])
def test_mismatch_raises(which, bad):
    built = tensors()
    called = list(tensors())
    idx = ("q", "cache", "out", "kv_new").index(which)
    called[idx] = bad(called[idx])
    with pytest.raises(ValueError):
        check(built, called)


def test_unfused_plan_rejects_kv_new():
    q, cache, out, kv = tensors()
    with pytest.raises(ValueError, match="kv_new"):
        check((q, cache, out, None), (q, cache, out, kv))


# ------------------------------------------------------------ the planner ---

def params(batch, hq, hkv, d, dtype=_lib.HEXKV_BF16, bias=0, max_seqlen=1 << 20, kv_new=True, partition=0):
    return _lib.AttendParams(dtype=dtype, batch=batch, q_len=1, q_heads=hq, kv_heads=hkv, head_dim=d,
                             softmax_scale=0.1, seqlen_bias=bias, max_seqlen=max_seqlen,
                             kv_new=0x1000 if kv_new else None, partition=partition)


def plan(p, lens):
    lib = _lib.load()
    c_lens = (ctypes.c_int32 * len(lens))(*lens)
    n, mp = ctypes.c_int32(), ctypes.c_int32()
    _lib.check(lib.hexkv_attend_plan(ctypes.byref(p), c_lens, None, 0, None, 0, ctypes.byref(n), ctypes.byref(mp)),
               "plan")
    items = (_lib.WorkItem * max(n.value, 1))()
    parts = (ctypes.c_int32 * (p.batch * p.q_heads))()
    n2, mp2 = ctypes.c_int32(), ctypes.c_int32()
    _lib.check(lib.hexkv_attend_plan(ctypes.byref(p), c_lens, items, n.value, parts, len(parts),
                                     ctypes.byref(n2), ctypes.byref(mp2)), "plan")
    assert (n2.value, mp2.value) == (n.value, mp.value)
    arr = np.array([[it.row, it.head_group, it.part, it.parts, it.first, it.count, it.len, it.heads]
                    for it in items[:n.value]], dtype=np.int64)
    return arr, np.array(parts[:]), mp.value


def group_of(hq, hkv):
    return next(g for g in (8, 4, 2, 1) if (hq // hkv) % g == 0)


def check_cover(arr, parts, lens, hq, hkv, bias=0, extra=1):
    groups = hq // group_of(hq, hkv)
    att = [n + bias + extra for n in lens]
    seen = {}
    for row, hg, part, nparts, first, count, length, _ in arr:
        assert 0 <= row < len(lens) and 0 <= hg < groups
        assert length == att[row] and 0 <= first and first + count <= length
        assert nparts == parts[row * groups + hg] and 0 <= part < nparts
        seen.setdefault((row, hg), []).append((part, first, count))
    for row in range(len(lens)):
        for hg in range(groups):
            spans = sorted(seen[(row, hg)], key=lambda x: x[1])
            assert [s[0] for s in spans] == list(range(len(spans))), "partitions numbered in position order"
            pos = 0
            for _, first, count in spans:
                assert first == pos
                pos += count
            assert pos == att[row]
            assert len(spans) == parts[row * groups + hg]


@pytest.mark.parametrize("lens,hq,hkv,d", [
    ([7897, 221, 4000, 1023, 1024, 1025, 0, 5000], 32, 8, 128),   # Llama-3-8B geometry, ragged
    ([3806, 538, 2000], 8, 1, 128),                                # Llama-2-70B TP-8 share
    ([512], 32, 4, 64),                                            # TinyLlama: no split
    ([100, 0, 3], 4, 4, 16),                                       # tiny fp32-style geometry
])
def test_plan_covers_every_position_once(lens, hq, hkv, d):
    p = params(len(lens), hq, hkv, d)
    arr, parts, max_parts = plan(p, lens)
    check_cover(arr, parts, lens, hq, hkv)
    assert max_parts == arr[:, 3].max()


def test_plan_order_full_chunks_then_tails_longest_first():
    lens = [5000, 3000, 2047, 4095]  # +1 attended each (fused append)
    p = params(len(lens), 32, 8, 128, partition=1024)
    arr, parts, _ = plan(p, lens)
    check_cover(arr, parts, lens, 32, 8)
    counts = arr[:, 5]
    full = counts == 1024
    last_full = np.nonzero(full)[0].max()
    assert full[:last_full + 1].all(), "every full chunk precedes every shorter one"
    tails = counts[last_full + 1:]
    assert (np.diff(tails) <= 0).all(), "shorter chunks from the longest down"
    # chunk index major across segments: the first items are chunk 0 of every segment
    groups = 32 // 4
    assert (arr[:len(lens) * groups, 2] == 0).all()


def test_plan_empty_rows_come_first_with_zero_counts():
    lens = [10, 0, 7]
    p = params(3, 8, 2, 64, kv_new=False)
    arr, parts, _ = plan(p, lens)
    check_cover(arr, parts, lens, 8, 2, extra=0)
    groups = 8 // 4
    assert (arr[:groups, 0] == 1).all() and (arr[:groups, 5] == 0).all()


def test_plan_chunk_regimes():
    # small call (< 4 MB read): one item per (row, head group), no merge
    arr, parts, mp = plan(params(1, 32, 4, 64, dtype=_lib.HEXKV_F16), [576])
    assert mp == 1 and len(arr) == 4
    # latency-bound (< 64 MB): about 240 items
    lens = [538 + 37 * i for i in range(32)]
    arr, _, mp = plan(params(32, 8, 1, 128), lens)
    assert 150 <= len(arr) <= 300 and mp > 1
    # bandwidth-bound: 896-position chunks, 1280 from a million positions up
    lens = [2000 - 10 * i for i in range(64)]
    arr, _, _ = plan(params(64, 32, 8, 128), lens)
    assert arr[:, 5].max() == 896
    lens = [8000 - 100 * i for i in range(64)]
    arr, _, _ = plan(params(64, 32, 8, 128), lens)
    assert arr[:, 5].max() == 1280


def test_plan_rejects_bad_requests():
    lib = _lib.load()
    n, mp = ctypes.c_int32(), ctypes.c_int32()
    lens = (ctypes.c_int32 * 2)(10, 20)
    p = params(2, 8, 2, 64, max_seqlen=15)  # 20 + 1 keys above max_seqlen
    assert lib.hexkv_attend_plan(ctypes.byref(p), lens, None, 0, None, 0, ctypes.byref(n), ctypes.byref(mp)) \
        == _lib.HEXKV_ERANGE
    p = params(2, 8, 2, 64)
    p.q_len = 2
    assert lib.hexkv_attend_plan(ctypes.byref(p), lens, None, 0, None, 0, ctypes.byref(n), ctypes.byref(mp)) \
        == _lib.HEXKV_EINVAL
    p = params(2, 8, 2, 64)
    items = (_lib.WorkItem * 1)()
    parts = (ctypes.c_int32 * 16)()
    assert lib.hexkv_attend_plan(ctypes.byref(p), lens, items, 1, parts, 16, ctypes.byref(n), ctypes.byref(mp)) \
        == _lib.HEXKV_EINVAL  # room for one item only


def plan_chunk(p, lens):
    lib = _lib.load()
    c_lens = (ctypes.c_int32 * len(lens))(*lens)
    chunk = ctypes.c_int32()
    rc = lib.hexkv_attend_plan_chunk(ctypes.byref(p), c_lens, ctypes.byref(chunk))
    return rc, chunk.value


@pytest.mark.parametrize("lens,hq,hkv,d,dtype", [
    ([576], 32, 4, 64, _lib.HEXKV_F16),                          # one chunk per segment
    ([538 + 37 * i for i in range(32)], 8, 1, 128, _lib.HEXKV_BF16),  # about 240 items
    ([2000 - 10 * i for i in range(64)], 32, 8, 128, _lib.HEXKV_BF16),
    ([8000 - 100 * i for i in range(64)], 32, 8, 128, _lib.HEXKV_BF16),
])
def test_plan_chunk_is_the_planners_chunk(lens, hq, hkv, d, dtype):
    """hexkv_attend_plan_chunk names the chunk the planner cuts with: no item
    is longer, every item but a segment's last has exactly that length, and
    planning with it passed as the partition gives the same list."""
    p = params(len(lens), hq, hkv, d, dtype=dtype)
    rc, chunk = plan_chunk(p, lens)
    assert rc == 0 and chunk > 0 and chunk % 64 == 0
    arr, parts, mp = plan(p, lens)
    assert arr[:, 5].max() <= chunk
    not_last = arr[:, 2] < arr[:, 3] - 1
    assert (arr[not_last, 5] == chunk).all()
    p2 = params(len(lens), hq, hkv, d, dtype=dtype, partition=chunk)
    arr2, parts2, mp2 = plan(p2, lens)
    assert np.array_equal(arr, arr2) and np.array_equal(parts, parts2) and mp == mp2
    assert plan_chunk(p2, lens) == (0, chunk)


def test_plan_takes_chunks_beyond_4096():
    """A work list may use chunks above the grid's 4096-position cap (the
    one-chunk-per-segment regime reaches them); the planner takes any
    positive multiple of 64."""
    lens = [9000, 100]
    p = params(2, 8, 2, 64, partition=8192)
    arr, parts, mp = plan(p, lens)
    check_cover(arr, parts, lens, 8, 2)
    assert mp == 2 and arr[:, 5].max() == 8192
    for bad in (100, -64):
        rc, _ = plan_chunk(params(2, 8, 2, 64, partition=bad), lens)
        assert rc == _lib.HEXKV_EINVAL
    rc, _ = plan_chunk(params(2, 8, 2, 64, max_seqlen=50), lens)
    assert rc == _lib.HEXKV_ERANGE


def check_order(arr):
    """Empty rows first, then every full chunk (all of one size), then the
    shorter last chunks from the longest down."""
    counts = arr[:, 5]
    empty = arr[:, 6] == 0
    n_empty = int(empty.sum())
    assert empty[:n_empty].all(), "empty rows come first"
    rest = counts[n_empty:]
    if len(rest) == 0:
        return
    chunk = rest.max()
    full = rest == chunk
    # full chunks are the segments' non-final pieces plus any last piece of exactly one chunk
    last_full = np.nonzero(full)[0].max() if full.any() else -1
    tails = rest[last_full + 1:]
    assert (np.diff(tails) <= 0).all(), "last chunks from the longest down"


@pytest.mark.parametrize("seed", range(40))
def test_random_plans(seed):
    """Random geometries, lengths (empty rows included), biases, chunk
    choices and append flags: every plan covers each attended position of
    each (row, head group) exactly once, in the dispatch order, and
    hexkv_attend_plan_chunk names the chunk it used."""
    rng = np.random.default_rng(7000 + seed)
    hkv = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([1, 2, 3, 4, 8, 16]))
    hq, d = hkv * group, int(rng.choice([16, 32, 64, 128, 256]))
    batch = int(rng.integers(1, 70))
    lens = [int(x) for x in rng.integers(0, 10000, batch)]
    if seed % 3 == 0:
        lens[int(rng.integers(batch))] = 0
    kv_new = bool(rng.integers(2))
    bias = int(rng.integers(0, 5))
    partition = int(rng.choice([0, 0, 64, 192, 1024, 4160, 8192]))
    dtype = int(rng.choice([_lib.HEXKV_F16, _lib.HEXKV_BF16, _lib.HEXKV_F32]))
    extra = 1 if kv_new else 0
    p = params(batch, hq, hkv, d, dtype=dtype, bias=bias, max_seqlen=max(lens) + bias + extra,
               kv_new=kv_new, partition=partition)
    arr, parts, mp = plan(p, lens)
    check_cover(arr, parts, lens, hq, hkv, bias=bias, extra=extra)
    check_order(arr)
    assert mp == max(1, int(arr[:, 3].max()))
    rc, chunk = plan_chunk(p, lens)
    assert rc == 0 and (partition == 0 or chunk == partition)
    assert arr[:, 5].max() <= chunk


def check_xcd_plan(arr, parts, lens, hq, hkv, xcds, bias=0, extra=1):
    """A plan for ``xcds`` XCDs: the real items cover every position once;
    every item of one (row, head group) sits at one index modulo ``xcds``
    (so they run on one XCD); each XCD's items keep the dispatch order;
    padding items (row = batch, all else zero) only end an XCD's share; the
    XCDs' positions differ by at most one segment's."""
    batch = len(lens)
    assert len(arr) % xcds == 0
    pad = arr[:, 0] == batch
    assert (arr[pad][:, 1:] == 0).all()
    check_cover(arr[~pad], parts, lens, hq, hkv, bias=bias, extra=extra)
    homes = {}
    for i in np.nonzero(~pad)[0]:
        homes.setdefault((int(arr[i, 0]), int(arr[i, 1])), set()).add(int(i) % xcds)
    assert all(len(h) == 1 for h in homes.values()), "a segment's items span XCDs"
    load = np.zeros(xcds, dtype=np.int64)
    for x in range(xcds):
        share = arr[x::xcds]
        col = share[:, 0] == batch
        if col.any():
            assert col[int(np.argmax(col)):].all(), "padding only at the end of an XCD's share"
        check_order(share[~col])
        load[x] = share[~col][:, 5].sum()
    # segments are dealt longest first to the least loaded XCD: the loads end
    # within one segment of each other
    assert load.max() - load.min() <= max(max(n + bias + extra for n in lens), 1)


@pytest.mark.parametrize("lens,hq,hkv,d", [
    ([7897, 221, 4000, 1023, 1024, 1025, 0, 5000], 32, 8, 128),   # Llama-3-8B geometry, ragged
    ([3806, 538, 2000], 8, 1, 128),                                # Llama-2-70B TP-8 share
    ([512], 32, 4, 64),                                            # TinyLlama
    ([100, 0, 3], 4, 4, 16),
])
@pytest.mark.parametrize("xcds", [1, 2, 8])
def test_xcd_plans(lens, hq, hkv, d, xcds):
    p = params(len(lens), hq, hkv, d)
    p.work_xcds = xcds
    rc, chunk = plan_chunk(p, lens)
    assert rc == 0
    arr, parts, mp = plan(p, lens)
    check_xcd_plan(arr, parts, lens, hq, hkv, xcds)
    # the same chunks as a plain plan cut at that chunk
    flat, flat_parts, flat_mp = plan(params(len(lens), hq, hkv, d, partition=chunk), lens)
    assert np.array_equal(parts, flat_parts) and mp == flat_mp
    if xcds == 1:
        assert np.array_equal(arr, flat), "one XCD: the plain order"


@pytest.mark.parametrize("seed", range(24))
def test_random_xcd_plans(seed):
    """Random geometries and lengths planned for 8 XCDs (and for a random
    count up to 64): the placement, cover and order rules of check_xcd_plan."""
    rng = np.random.default_rng(9000 + seed)
    hkv = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([1, 2, 4, 8]))
    hq, d = hkv * group, int(rng.choice([64, 128]))
    batch = int(rng.integers(1, 70))
    lens = [int(x) for x in rng.integers(0, 9000, batch)]
    kv_new = bool(rng.integers(2))
    extra = 1 if kv_new else 0
    partition = int(rng.choice([0, 0, 64, 320, 1280]))
    for xcds in (8, int(rng.integers(2, 65))):
        p = params(batch, hq, hkv, d, max_seqlen=max(lens) + extra, kv_new=kv_new, partition=partition)
        p.work_xcds = xcds
        arr, parts, _ = plan(p, lens)
        check_xcd_plan(arr, parts, lens, hq, hkv, xcds, extra=extra)


def test_xcd_plan_rejects_bad_counts():
    lib = _lib.load()
    n, mp = ctypes.c_int32(), ctypes.c_int32()
    lens = (ctypes.c_int32 * 2)(10, 20)
    for bad in (-1, 65):
        p = params(2, 8, 2, 64)
        p.work_xcds = bad
        assert lib.hexkv_attend_plan(ctypes.byref(p), lens, None, 0, None, 0, ctypes.byref(n),
                                     ctypes.byref(mp)) == _lib.HEXKV_EINVAL
    # more (row, head group) segments than the merge has counters for
    many = 20000
    big = (ctypes.c_int32 * many)(*([1] * many))
    p = params(many, 8, 8, 64)  # 8 segments per row
    assert lib.hexkv_attend_plan(ctypes.byref(p), big, None, 0, None, 0, ctypes.byref(n),
                                 ctypes.byref(mp)) == _lib.HEXKV_OK
    p.work_xcds = 8
    assert lib.hexkv_attend_plan(ctypes.byref(p), big, None, 0, None, 0, ctypes.byref(n),
                                 ctypes.byref(mp)) == _lib.HEXKV_EINVAL
    assert b"segments" in lib.hexkv_last_error()


def test_small_calls_split_when_merged_in_kernel():
    """Below 4 MB read a call is one item per segment with a second-kernel
    merge (the merge launch would cost more than the split saves), but split
    into pieces of about a twelfth of the longest row, 64 positions at least,
    when planned for the XCDs (merged in the attention kernel)."""
    p = params(1, 32, 4, 64, dtype=_lib.HEXKV_F16)
    arr, _, mp = plan(p, [576])
    assert mp == 1 and len(arr) == 4
    p.work_xcds = 8
    rc, chunk = plan_chunk(p, [576])
    assert rc == 0 and chunk == 64
    arr, parts, mp = plan(p, [576])
    assert mp == 10 and (parts[:4] == 10).all()
    check_xcd_plan(arr, parts, [576], 32, 4, 8)
    assert len(arr) == 80  # 4 XCDs with one segment's 10 items, 4 with padding only
    rc, chunk = plan_chunk(p, [4000])
    assert rc == 0 and chunk == 384


# ------------------------------------------------------- row-block lists ---

def rows_params(batch, hq, hkv, dtype=_lib.HEXKV_BF16, partition=0, xcds=8):
    p = params(batch, hq, hkv, 128, dtype=dtype, partition=partition)
    p.kernel, p.work_xcds = _lib.KERNELS["rows"], xcds
    return p


def rows_block(hq, hkv):
    group = hq // hkv
    if group > 1:
        return 2
    return next(hb for hb in (8, 4, 2) if hkv % hb == 0)


@pytest.mark.parametrize("lens,hq,hkv", [
    ([7897, 221, 4000, 1023, 1024, 1025, 0, 5000], 32, 8),  # Llama-3-8B geometry: 2 KV heads per item
    ([2000, 300, 1500, 256, 64, 0, 1999, 777], 32, 32),     # Llama-2-7B geometry: 8 KV heads per item
    ([900, 17, 3], 8, 4),                                   # group 2
    ([513, 1, 60], 4, 4),                                   # group 1, 4 KV heads: 4 per item
])
def test_row_block_plans_cover_every_position_once(lens, hq, hkv):
    """Row-block lists: segments of hb adjacent KV heads (hb * group query
    heads, recorded in every item), every attended position of every segment
    once, each segment on one XCD, at most 64 pieces per segment."""
    pieces = -(-(max(lens) + 1) // 64)  # 64 pieces of the longest row at most
    finest = max(16, (pieces + 15) // 16 * 16)
    for partition in (0, finest, 3 * finest):
        p = rows_params(len(lens), hq, hkv, partition=partition)
        arr, parts, max_parts = plan(p, lens)
        heads = rows_block(hq, hkv) * (hq // hkv)
        real = arr[arr[:, 0] < len(lens)]
        assert (real[:, 7] == heads).all(), "items record their head-group size"
        groups = hq // heads
        att = [n + 1 for n in lens]
        seen = {}
        for i, (row, hg, part, nparts, first, count, length, _) in enumerate(arr):
            if row >= len(lens):
                continue  # padding
            assert 0 <= hg < groups and length == att[row] and nparts == parts[row * groups + hg]
            seen.setdefault((row, hg), []).append((first, count, i % 8))
        for row in range(len(lens)):
            for hg in range(groups):
                spans = sorted(seen[(row, hg)])
                assert len({x for _, _, x in spans}) == 1, "a segment's items share one XCD"
                pos = 0
                for first, count, _ in spans:
                    assert first == pos
                    pos += count
                assert pos == att[row]
        assert max_parts <= 64


def full_chunks_per_xcd(arr, batch, chunk, xcds=8):
    """Full chunks (count == chunk) in each XCD's share (item i runs on XCD i % xcds)."""
    full = [0] * xcds
    for i, it in enumerate(arr):
        if it[0] < batch and it[5] == chunk:
            full[i % xcds] += 1
    return full


def test_row_block_chunk_rule():
    """The smallest chunk (a multiple of 16) at which no XCD's share holds
    more than 27/32 of its 32 CUs' workgroup slots (4 per CU with 4 query
    heads per KV head, 5 otherwise) in full chunks, with items of at least
    448 KiB and at most 64 pieces per row: at Llama-3-8B's decode steps
    ~1,100 items (1 KB per position), at Llama-2-7B's 112-position items (4
    KB per position)."""
    from hexgen2_amd.workloads import workload
    for name, hq, hkv, dtype, limit, floor, window in (
            ("llama3-8b", 32, 8, _lib.HEXKV_BF16, 108, 448, (1000, 1200)),
            ("llama2-7b", 32, 32, _lib.HEXKV_F16, 135, 112, (330, 480))):
        w = workload(name)
        for t in (0, w.decode_steps // 2, w.decode_steps - 1):
            lens = [n + t for n in w.lens]
            p = rows_params(w.batch, hq, hkv, dtype=dtype)
            rc, chunk = plan_chunk(p, lens)
            assert rc == 0 and chunk % 16 == 0 and chunk >= floor
            arr, _, max_parts = plan(p, lens)
            assert window[0] <= int((arr[:, 0] < w.batch).sum()) <= window[1], (name, t, len(arr))
            assert max_parts <= 64
            assert max(full_chunks_per_xcd(arr, w.batch, chunk)) <= limit
            if chunk > floor:  # one step finer would overfill a share
                finer = rows_params(w.batch, hq, hkv, dtype=dtype, partition=chunk - 16)
                arr2, _, _ = plan(finer, lens)
                assert max(full_chunks_per_xcd(arr2, w.batch, chunk - 16)) > limit, (name, t, chunk)
    # one long row: the chunk grows so that the row has at most 64 pieces
    p = rows_params(1, 32, 8)
    for n in (100000, 1036, 1500, 4095):
        rc, chunk = plan_chunk(p, [n])
        assert rc == 0 and chunk % 16 == 0 and (n + 1 + chunk - 1) // chunk <= 64, (n, chunk)
    # a forced partition that would need more pieces is refused
    p = rows_params(1, 32, 8, partition=16)
    rc, _ = plan_chunk(p, [5000])
    assert rc == _lib.HEXKV_EUNSUPPORTED


@pytest.mark.parametrize("hq,hkv", [(32, 8), (64, 16), (16, 4), (32, 16)])
def test_row_block_shares_match_xcd_parity(hq, hkv):
    """Two-head blocks (512 bytes of K and of V at 16 bits, head_dim 128):
    block hb's slices have address bit 9 = hb & 1, and an XCD reads slices
    of its own parity faster.  The planner's deal gives XCD x only blocks of
    x's parity (XCD x's items sit at indices i with i % 8 == x)."""
    rng = np.random.default_rng(hkv)
    for _ in range(3):
        lens = [int(n) for n in rng.integers(128, 8192, 64)]
        arr, _, _ = plan(rows_params(64, hq, hkv), lens)
        for i, it in enumerate(arr):
            if it[0] < 64:
                assert (it[1] & 1) == (i % 8) & 1, (i, it)


def plan_kernel(p, lens):
    lib = _lib.load()
    c_lens = (ctypes.c_int32 * len(lens))(*lens)
    k = ctypes.c_int32()
    rc = lib.hexkv_attend_plan_kernel(ctypes.byref(p), c_lens, ctypes.byref(k))
    return rc, k.value


def test_plan_kernel_choice():
    """hexkv_attend_plan_kernel: the row-block kernel for "auto" on calls of
    64 MB or more that fit it and are planned for the XCDs; AUTO's own
    choice otherwise; an explicit kernel as given."""
    from hexgen2_amd.workloads import workload
    K = _lib.KERNELS
    w = workload("llama3-8b")
    p = params(w.batch, 32, 8, 128)
    p.work_xcds = 8
    assert plan_kernel(p, w.lens) == (0, K["rows"])
    p.work_xcds = 0  # merged by a second launch: not the row-block kernel
    assert plan_kernel(p, w.lens) == (0, K["valu"])
    p.work_xcds, p.kernel = 8, K["valu"]
    assert plan_kernel(p, w.lens) == (0, K["valu"])
    w = workload("llama2-7b")
    p = params(w.batch, 32, 32, 128, dtype=_lib.HEXKV_F16)
    p.work_xcds = 8
    assert plan_kernel(p, w.lens) == (0, K["rows"])
    # small calls, one KV head, fp32, head_dim 64: AUTO's own choice
    p = params(2, 32, 8, 128)
    p.work_xcds = 8
    assert plan_kernel(p, [100, 200]) == (0, K["valu"])
    w = workload("llama2-70b-tp8")
    p = params(w.batch, 8, 1, 128)
    p.work_xcds = 8
    assert plan_kernel(p, w.lens) == (0, K["mfma"])
    p = params(64, 32, 8, 128, dtype=_lib.HEXKV_F32)
    p.work_xcds = 8
    assert plan_kernel(p, [8000] * 64) == (0, K["valu"])
    p = params(64, 32, 8, 64)
    p.work_xcds = 8
    assert plan_kernel(p, [8000] * 64)[1] != K["rows"]
