"""Host logic of the legacy-format wrappers, without a GPU: the block
description ``kv_formats._as_block`` gives of a tensor must address exactly
the tensor's bytes, in row-major order.  Checked by gathering bytes from the
tensor's storage through the block and comparing with ``t.contiguous()``."""
import ctypes

import numpy as np
import pytest
import torch

from hexgen2_amd import _lib, kv_formats as kvf


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
    fields, c = kvf._block(t, split=1)
    assert c.is_contiguous() and _lib.Block(*fields).width == 4 * 6 * 4


def test_layout_cache_keeps_each_tensors_address():
    big = torch.arange(2 * 5 * 8, dtype=torch.float32).reshape(2, 5, 8)
    a, b = kvf._as_block(big[0, :3]), kvf._as_block(big[1, :3])  # same shape and stride
    assert (a.width, a.height, a.depth) == (b.width, b.height, b.depth)
    assert b.data - a.data == 5 * 8 * 4
    np.testing.assert_array_equal(gather(big[1, :3], b), expect(big[1, :3]))


def test_block_array_is_the_c_struct_array():
    fields = [(0x1000 * (i + 1), 16 * i, i, 2 * i, 64, 4096) for i in range(5)]
    arr = kvf._block_array(fields)
    assert ctypes.sizeof(_lib.Block) == 6 * 8
    for i, f in enumerate(fields):
        b = arr[i]
        assert (b.data, b.width, b.height, b.depth, b.row_pitch, b.slice_pitch) == f


# The wrappers on host tensors with the library call captured: every block
# handed to the C ABI must address exactly the bytes of its tensor.

class _Capture:
    def __init__(self):
        self.calls = []

    @staticmethod
    def _fields(blocks, n):
        return [(b.data, b.width, b.height, b.depth, b.row_pitch, b.slice_pitch) for b in
                (blocks[i] for i in range(n))]

    def hexkv_flat_concat(self, blocks, n, dst, stream):
        self.calls.append(("flat", self._fields(blocks, n), dst))
        return 0

    def hexkv_batch_pad(self, blocks, n_layers, n_req, dst, max_rows, stream):
        self.calls.append(("batch", self._fields(blocks, n_layers * n_req), [dst[l] for l in range(n_layers)],
                           max_rows))
        return 0

    def hexkv_head_concat(self, blocks, n_layers, n_shards, dst, stream):
        self.calls.append(("concat", self._fields(blocks, n_layers * n_shards), [dst[l] for l in range(n_layers)]))
        return 0


@pytest.fixture
def captured(monkeypatch):
    cap = _Capture()
    monkeypatch.setattr(kvf._lib, "load", lambda: cap)
    monkeypatch.setattr(kvf, "_require_device", lambda *t: None)
    monkeypatch.setattr(kvf, "_stream", lambda t: None)
    return cap


def _bytes_at(t: torch.Tensor, fields) -> np.ndarray:
    return gather(t, _lib.Block(*fields))


def test_batch_pad_blocks_address_every_request(captured):
    g = torch.Generator().manual_seed(0)
    lens = [5, 9, 1, 7]
    cache = torch.randn((3, 4, 12, 2, 3, 4), generator=g).to(torch.float16)
    odd = torch.randn((3, 1, 6, 4, 3, 2), generator=g).to(torch.float16).permute(0, 1, 2, 5, 4, 3)
    dicts = [{l: cache[l, i:i + 1, :n] for l in range(3)} for i, n in enumerate(lens)]
    dicts.append({l: odd[l] for l in range(3)})  # rows (dims 2+) not contiguous: copied first
    out = kvf.batch_key_value_memory_dicts(dicts)
    (kind, fields, dst, max_rows), = captured.calls
    assert kind == "batch" and max_rows == 9 and len(fields) == 3 * 5
    assert dst == [out[l].data_ptr() for l in range(3)]
    for l in range(3):
        for i, d in enumerate(dicts):
            f = fields[l * 5 + i]
            t = d[l]
            assert (f[1], f[2], f[3]) == (2 * 3 * 4 * 2, t.shape[1], t.shape[0])
            if i < 4:
                np.testing.assert_array_equal(_bytes_at(t, f), expect(t))
            else:  # a contiguous copy was described; it holds the same values
                assert f[0] != t.data_ptr() and f[4] == 2 * 3 * 4 * 2


def test_head_concat_blocks_address_every_shard(captured):
    g = torch.Generator().manual_seed(1)
    shards_t = torch.randn((4, 2, 3, 10, 2, 1, 8), generator=g).to(torch.bfloat16)
    shards = [{l: shards_t[j, l] for l in range(2)} for j in range(4)]
    out = kvf.concat_dicts(shards)
    (kind, fields, dst), = captured.calls
    assert kind == "concat" and len(fields) == 2 * 4 and dst == [out[l].data_ptr() for l in range(2)]
    for l in range(2):
        for j in range(4):
            np.testing.assert_array_equal(_bytes_at(shards[j][l], fields[l * 4 + j]), expect(shards[j][l]))


def test_flat_concat_blocks_address_every_tensor(captured):
    big = torch.arange(2 * 4 * 10 * 6, dtype=torch.float32).reshape(2, 4, 10, 6)
    tensors = [big[0, :, :7], big[1, 1:3], big[0, :, :, 2:5]]
    out = torch.empty(sum(t.numel() for t in tensors))
    kvf.flat_concat(tensors, out=out)
    (kind, fields, dst), = captured.calls
    assert kind == "flat" and dst == out.data_ptr() and len(fields) == 3
    for t, f in zip(tensors, fields):
        np.testing.assert_array_equal(_bytes_at(t, f), expect(t))
