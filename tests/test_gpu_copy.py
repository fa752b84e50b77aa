"""GPU parity of pack / unpack / append against the oracle: bit-exact.

Tensors are compared as integer views of their bytes, so NaN payloads and
signed zeros count too.  Destinations are sentinel-filled to prove that no
byte outside the live rows is written.
"""
import numpy as np
import pytest
import torch

from hexgen2_amd import ops
from oracle import kv_oracle as oracle

pytestmark = pytest.mark.gpu

INT_VIEW = {torch.float16: torch.int16, torch.bfloat16: torch.int16, torch.float32: torch.int32}


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(INT_VIEW[t.dtype]).numpy()


def rand_layers(n_layers, batch, cap, row_shape, dtype, seed, device):
    g = torch.Generator(device=device).manual_seed(seed)
    return [torch.randn((batch, cap, *row_shape), generator=g, device=device).to(dtype)
            for _ in range(n_layers)]


CASES = [
    # (n_layers, lens, capacity, row_shape, dtype)
    (2, [16], 24, (2, 4, 16), torch.float32),          # tiny-llama geometry, batch 1
    (22, [512], 640, (2, 4, 64), torch.float16),       # TinyLlama geometry
    (3, [256, 2048, 1000, 0, 1], 2048, (2, 32, 128), torch.float16),  # MHA rows, ragged + empty
    (4, [512, 4096, 777, 3], 4128, (2, 1, 128), torch.bfloat16),      # 1 KV head (TP-8 share)
    (2, [128, 8192, 4000, 129], 8448, (2, 8, 128), torch.bfloat16),   # Llama-3-8B geometry
    (2, [5, 0, 3], 7, (2, 1, 3), torch.float16),       # 12-byte rows: 4-byte vector path
    (1, [0, 0], 4, (2, 2, 8), torch.float32),          # nothing live
]


@pytest.mark.parametrize("n_layers,lens,cap,row_shape,dtype", CASES)
def test_pack_unpack_bit_exact(device, n_layers, lens, cap, row_shape, dtype):
    print(f"pack/unpack layers={n_layers} lens={lens} cap={cap} row={row_shape} {dtype}", flush=True)
    layers = rand_layers(n_layers, len(lens), cap, row_shape, dtype, 11, device)
    packed = ops.pack_live(layers, lens)
    torch.cuda.synchronize()
    expect = oracle.pack([bits(t) for t in layers], lens)
    np.testing.assert_array_equal(bits(packed), expect)
    # determinism: a second pack is byte-identical
    np.testing.assert_array_equal(bits(ops.pack_live(layers, lens)), expect)

    sentinel = torch.full((len(lens), cap, *row_shape), -3.0, dtype=dtype, device=device)
    dst = [sentinel.clone() for _ in range(n_layers)]
    ops.unpack_live(packed, dst, lens)
    torch.cuda.synchronize()
    want = oracle.unpack(expect, [bits(sentinel)] * n_layers, lens)
    for l in range(n_layers):
        np.testing.assert_array_equal(bits(dst[l]), want[l])


def test_pack_many_layers_and_sequences_split_launches(device):
    # 100 layers > 96 per launch and 300 sequences > 256 per launch
    lens = [int(x) for x in np.random.default_rng(0).integers(0, 6, size=300)]
    layers = rand_layers(100, 300, 6, (2, 1, 8), torch.float16, 3, device)
    packed = ops.pack_live(layers, lens)
    expect = oracle.pack([bits(t) for t in layers], lens)
    np.testing.assert_array_equal(bits(packed), expect)
    dst = [torch.zeros_like(layers[0]) for _ in range(100)]
    ops.unpack_live(packed, dst, lens)
    want = oracle.unpack(expect, [bits(dst[0])] * 100, lens)
    for l in (0, 57, 95, 96, 99):
        np.testing.assert_array_equal(bits(dst[l]), want[l])


@pytest.mark.parametrize("n_layers,batch", [(32, 16), (33, 16), (32, 17), (100, 10)])
def test_launches_around_the_small_argument_block(device, n_layers, batch):
    # launches of up to 32 layers and 16 sequences carry a small kernel-argument
    # block, larger ones the full one; 100 layers = a full launch of 96, then 4
    print(f"argument block layers={n_layers} batch={batch}", flush=True)
    lens = [int(x) for x in np.random.default_rng(n_layers + batch).integers(0, 9, size=batch)]
    layers = rand_layers(n_layers, batch, 9, (2, 1, 8), torch.float16, 4, device)
    packed = ops.pack_live(layers, lens)
    expect = oracle.pack([bits(t) for t in layers], lens)
    np.testing.assert_array_equal(bits(packed), expect)
    dst = [torch.full_like(layers[0], 5.0) for _ in range(n_layers)]
    ops.unpack_live(packed, dst, lens)
    want = oracle.unpack(expect, [bits(dst[0])] * n_layers, lens)
    for l in range(n_layers):
        np.testing.assert_array_equal(bits(dst[l]), want[l])


def test_launches_follow_the_current_stream(device):
    layers = rand_layers(3, 2, 6, (2, 1, 8), torch.float16, 8, device)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        assert (ops._stream(layers[0]).value or 0) == side.cuda_stream
        packed = ops.pack_live(layers, [6, 2])
    # the default stream's handle is 0, which ctypes reads back as None
    assert (ops._stream(layers[0]).value or 0) == torch.cuda.current_stream().cuda_stream
    side.synchronize()
    np.testing.assert_array_equal(bits(packed), oracle.pack([bits(t) for t in layers], [6, 2]))


def test_pack_into_per_layer_views_and_strided_batch(device):
    # caches that are batch slices of a larger allocation (batch_size_offset)
    big = rand_layers(2, 5, 10, (2, 2, 16), torch.bfloat16, 5, device)
    layers = [t[1:4] for t in big]  # batch stride = 10 rows, 3 sequences
    lens = [10, 0, 4]
    out = [torch.empty((14, 2, 2, 16), dtype=torch.bfloat16, device=device) for _ in range(2)]
    ops.pack_live(layers, lens, out=out)
    expect = oracle.pack([bits(t) for t in layers], lens)
    for l in range(2):
        np.testing.assert_array_equal(bits(out[l]), expect[l])


def test_stacked_tensors_match_layer_lists(device):
    # one [n_layers, B, S, *row] tensor (here a strided view: capacity 9 of 12)
    # and a stacked [n_layers, T, *row] packed tensor address the same bytes
    # as the per-layer lists
    g = torch.Generator(device=device).manual_seed(9)
    big = torch.randn((3, 4, 12, 2, 2, 16), generator=g, device=device).to(torch.bfloat16)
    cache = big[:, :, :9]
    lens = [9, 0, 2, 5]
    packed = torch.empty((3, 16, 2, 2, 16), dtype=torch.bfloat16, device=device)
    ops.pack_live(cache, lens, out=packed)
    expect = oracle.pack([bits(cache[l]) for l in range(3)], lens)
    np.testing.assert_array_equal(bits(packed), expect)
    dst = torch.full((3, 4, 9, 2, 2, 16), 7.0, dtype=torch.bfloat16, device=device)
    sentinel = bits(dst[0])
    ops.unpack_live(packed, dst, lens)
    want = oracle.unpack(expect, [sentinel] * 3, lens)
    for l in range(3):
        np.testing.assert_array_equal(bits(dst[l]), want[l])
    with pytest.raises(ValueError, match="contiguous"):
        ops.pack_live(cache, lens, out=packed[:, :8])


def test_unaligned_pointer_uses_narrow_vectors(device):
    base = torch.randn(2 * 9 * 16 + 2, device=device).to(torch.float16)
    cache = base[2:].view(2, 9, 2, 1, 8)  # 4-byte aligned, not 16-byte aligned
    assert cache.data_ptr() % 16 != 0
    packed = ops.pack_live([cache], [9, 4])
    np.testing.assert_array_equal(bits(packed), oracle.pack([bits(cache)], [9, 4]))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_append_per_sequence_positions(device, dtype):
    g = torch.Generator().manual_seed(2)
    cache = torch.randn((4, 12, 2, 8, 16), generator=g).to(dtype).to(device)
    kv = torch.randn((4, 2, 8, 16), generator=g).to(dtype).to(device)
    before = bits(cache)
    positions = torch.tensor([0, 11, 5, 7], dtype=torch.int32, device=device)
    ops.append_kv(cache, kv, positions)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(cache), oracle.append(before, bits(kv), [0, 11, 5, 7]))
    # uniform position via bias, on a batch slice of the cache
    before = bits(cache)
    ops.append_kv(cache[1:3], kv[:2].contiguous(), position_bias=3)
    want = before.copy()
    want[1:3] = oracle.append(before[1:3], bits(kv[:2]), [3, 3])
    np.testing.assert_array_equal(bits(cache), want)


def test_append_out_of_range_rows_are_skipped_on_device(device):
    """Positions read on the device outside [0, capacity) are not written,
    and the status word reports it (ValueError at the next check); an
    in-range append leaves the status clear."""
    ops.device_status()  # start clear
    cache = torch.zeros((3, 4, 2, 1, 8), dtype=torch.float16, device=device)
    kv = torch.ones((3, 2, 1, 8), dtype=torch.float16, device=device)
    ops.append_kv(cache, kv, torch.tensor([4, -1, 2], dtype=torch.int32, device=device))
    torch.cuda.synchronize()
    got = cache.cpu()
    assert (got[0] == 0).all() and (got[1] == 0).all()
    assert (got[2, 2] == 1).all() and got[2].sum() == 16
    with pytest.raises(ValueError, match="append position"):
        ops.check_device_status()
    ops.append_kv(cache, kv, torch.tensor([3, 0, 1], dtype=torch.int32, device=device))
    ops.check_device_status()  # cleared by the check above; nothing new


def test_host_validation_rejects_bad_lengths_before_launch(device):
    layers = rand_layers(1, 2, 4, (2, 1, 8), torch.float16, 0, device)
    with pytest.raises(ValueError, match="outside"):
        ops.pack_live(layers, [5, 1])
    with pytest.raises(ValueError, match="outside"):
        ops.pack_live(layers, [-1, 1])
    with pytest.raises(ValueError):
        ops.append_kv(layers[0], torch.zeros((2, 16), dtype=torch.float16, device=device), position_bias=4)
