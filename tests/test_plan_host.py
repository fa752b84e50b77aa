"""Host-side checks of AttendPlan's per-call geometry comparison (no GPU).

An AttendPlan patches only addresses into a parameter block built once, so a
call with a tensor of another shape, stride, dtype or device, or a short or
non-contiguous kv_new, must raise ValueError before anything is launched.
The comparison is a pure function of tensor metadata; it is exercised here on
CPU tensors."""
import pytest
import torch

from hexgen2_amd import ops


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
