"""hexkv_attend_noalloc (static per-GPU scratch, no allocation) against
hexkv_attend (caller's workspace), both called through the C ABI.

The two entry points run the same kernels with the same partitioning (the
library's grid, or one host-planned work list for both, its split rows
merged by a second kernel or, planned for the device's XCDs, inside the
attention kernel with arrival counters at the front of the workspace / the
scratch), so their outputs must agree bit for bit (and the fused append must
write the same cache bytes); each output is also checked against the float64
oracle (bf16 8e-3, fp16 2e-3 max-abs).  Two calls in a row, the second with
fewer rows and shorter lengths, so stale partials or counters of the first
call in the shared scratch would show.  A request beyond the scratch is
refused with HEXKV_EWORKSPACE before anything is launched.
"""
import ctypes

import numpy as np
import pytest
import torch

from hexgen2_amd import _lib, ops
from oracle import kv_oracle as oracle

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-3, torch.bfloat16: 8e-3}


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy()


def stream_of(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def both(q, cache, lens, kv_new, kernel, listed=None):
    """(workspace output, no-alloc output, cache after each) of one call;
    ``listed`` "xcd" or "two-launch": both calls run the same host-planned
    work list of 128-position items (its device buffers are the caller's
    inputs), merged in the attention kernel or by a second one."""
    lib = _lib.load()
    ops.device_status()  # clear flags earlier tests may have raised on purpose
    seqlens = torch.tensor(lens, dtype=torch.int32, device=q.device)
    max_seqlen = max(lens) + 1
    c_ws, c_na = cache.clone(), cache.clone()
    o_ws, o_na = torch.full_like(q, 7.0), torch.full_like(q, -7.0)
    # The work list is cut into 128-position chunks so that both calls split.
    p = ops._attend_params(q, c_ws, o_ws, seqlens, 0, max_seqlen, kv_new, False, None, 128 if listed else 0,
                           kernel)
    work = ops._plan_work(p, lens, q.device, single_launch=listed == "xcd") if listed else None
    if work:
        work.apply(p)
        assert (work.xcds > 0) == (listed == "xcd")
    need = lib.hexkv_attend_workspace_bytes(ctypes.byref(p))
    assert 0 < need <= _lib.NOALLOC_SCRATCH_BYTES
    ws = torch.zeros(need, dtype=torch.uint8, device=q.device)  # counters zero before first use
    _lib.check(lib.hexkv_attend(ctypes.byref(p), ctypes.c_void_p(ws.data_ptr()), need, stream_of(q)),
               "hexkv_attend")
    p = ops._attend_params(q, c_na, o_na, seqlens, 0, max_seqlen, kv_new, False, None, 0, kernel)
    if work:
        work.apply(p)
    _lib.check(lib.hexkv_attend_noalloc(ctypes.byref(p), stream_of(q)), "hexkv_attend_noalloc")
    torch.cuda.synchronize()
    status = ops.device_status()
    print(f"  device status {status:#x}", flush=True)
    assert status & _lib.STATUS_ERRORS == 0
    return o_ws, o_na, c_ws, c_na


@pytest.mark.parametrize("listed", [None, "two-launch", "xcd"], ids=["grid", "work_list", "xcd_work_list"])
@pytest.mark.parametrize("dtype,hq,hkv,d,kernel", [(torch.bfloat16, 32, 8, 128, "valu"),
                                                   (torch.bfloat16, 8, 1, 128, "mfma"),
                                                   (torch.float16, 32, 4, 64, "mfma")])
def test_noalloc_matches_workspace_entry_point(device, dtype, hq, hkv, d, kernel, listed):
    compare_entry_points(device, dtype, hq, hkv, d, kernel, listed)


def test_noalloc_row_block_matches_workspace_entry_point(device):
    """The row-block kernel (work lists planned for the XCDs only) through
    both entry points."""
    compare_entry_points(device, torch.bfloat16, 32, 8, 128, "rows", "xcd")


def compare_entry_points(device, dtype, hq, hkv, d, kernel, listed):
    g = torch.Generator(device=device).manual_seed(31)
    calls = [[5000, 17, 3000, 1, 2048, 700, 4095, 64, 1500, 333, 2600, 4000],  # up to 40 partitions
             [900, 3, 650]]                                                   # second call: smaller
    for i, lens in enumerate(calls):
        print(f"noalloc {dtype} {hq}/{hkv}/{d} {kernel} list={listed} call {i}: {len(lens)} rows", flush=True)
        cap = max(lens) + 8
        q = torch.randn((len(lens), 1, hq, d), generator=g, device=device).to(dtype)
        cache = torch.randn((len(lens), cap, 2, hkv, d), generator=g, device=device).to(dtype)
        kv_new = torch.randn((len(lens), 2, hkv, d), generator=g, device=device).to(dtype)
        o_ws, o_na, c_ws, c_na = both(q, cache, lens, kv_new, kernel, listed)
        assert np.array_equal(bits(o_na), bits(o_ws)), f"call {i}: outputs differ"
        assert np.array_equal(bits(c_na), bits(c_ws)), f"call {i}: appended caches differ"
        np.testing.assert_array_equal(bits(c_na), oracle.append(bits(cache), bits(kv_new), lens))
        ref = oracle.attend(q.cpu().double().numpy(), c_na.cpu().double().numpy(), [n + 1 for n in lens])
        err = float(np.abs(o_na.cpu().double().numpy() - ref).max())
        assert err <= TOL[dtype], f"call {i}: max-abs {err}"


def test_noalloc_refuses_beyond_scratch(device):
    # 64 rows x 32 heads x 64 partitions of 128 positions: 68 MB of partials
    q = torch.zeros((64, 1, 32, 128), dtype=torch.bfloat16, device=device)
    cache = torch.zeros((64, 8192, 2, 1, 128), dtype=torch.bfloat16, device=device)
    out = torch.empty_like(q)
    with pytest.raises(ValueError, match="static scratch"):
        ops.decode_attention_noalloc(q, cache, out, max_seqlen=8192, seqlen_bias=8192, partition=128)
