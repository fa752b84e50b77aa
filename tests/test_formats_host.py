"""Host logic of the legacy-format wrappers, without a GPU: the block
description ``kv_formats._as_block`` gives of a tensor must address exactly
the tensor's bytes, in row-major order.  Checked by gathering bytes from the
tensor's storage through the block and comparing with ``t.contiguous()``."""
import numpy as np
import pytest
import torch

from hexgen2_amd import kv_formats as kvf


def gather(t: torch.Tensor, b) -> np.ndarray:
    storage = np.frombuffer(bytes(t.untyped_storage()), dtype=np.uint8)
    base = b.data - t.untyped_storage().data_ptr() if b.data else 0
    out = []
    for k in range(b.depth):
        for r in range(b.height):
            start = base + k * b.slice_pitch + r * b.row_pitch
            out.append(storage[start:start + b.width])
    return np.concatenate(out) if out else np.zeros(0, np.uint8)


def expect(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.uint8).reshape(-1).numpy() if t.numel() else np.zeros(0, np.uint8)


def views():
    big = torch.arange(3 * 4 * 10 * 2 * 3 * 8, dtype=torch.float16).reshape(3, 4, 10, 2, 3, 8)
    return {
        "contiguous": big[0],
        "cache slice [:, :L]": big[1, :, :7],
        "batch slice": big[2, 1:3],
        "head slice": big[0, :, :5, :, :2],
        "one head": big[1, :, :, :, 1:2],
        "layer stack view": big[:, :, :6],
        "size-1 batch": big[0, :1, :9],
        "expanded": torch.arange(16, dtype=torch.float32).reshape(1, 16).expand(5, 16),
        "empty": big[0, :, :0],
    }


@pytest.mark.parametrize("name", list(views()))
def test_default_block_addresses_the_tensor(name):
    t = views()[name]
    b = kvf._as_block(t)
    if b is None:
        pytest.skip("layout needs more than two strided levels (made contiguous first)")
    assert b.width * b.height * b.depth == t.numel() * t.element_size()
    np.testing.assert_array_equal(gather(t, b), expect(t))


@pytest.mark.parametrize("name", list(views()))
@pytest.mark.parametrize("split", [1, 2, 3])
def test_split_blocks_have_rows_of_the_trailing_dims(name, split):
    t = views()[name]
    if t.dim() <= split:
        return
    b = kvf._as_block(t, split)
    if b is None:  # rows not contiguous, or the outer dims need three levels
        assert not t[(0,) * split].is_contiguous() or split > 2
        return
    if t.numel():
        assert b.width == int(np.prod(t.shape[split:])) * t.element_size()
    np.testing.assert_array_equal(gather(t, b), expect(t))


def test_non_contiguous_rows_have_no_block():
    t = torch.zeros((4, 6, 5)).permute(2, 0, 1)
    assert kvf._as_block(t, split=1) is None
    b, c = kvf._block(t, split=1)
    assert c.is_contiguous() and b.width == 4 * 6 * 4
