"""GPU parity of the legacy KV formats (hexgen2_amd.kv_formats) against the
oracle, bit-exact: the flat KV packet and its two-process wire exchange,
zero-padded request batching and the tensor-parallel head concatenation.

Geometries: the reference scripts' own example shapes (scaled where noted),
the Llama geometries of the data path, strided cache views, layouts that
force the 4- and 2-byte vector paths, empty requests and shards, rows longer
than one tile, and more spans than one launch carries."""
from datetime import timedelta
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.distributed as dist
import torch.multiprocessing as mp

from hexgen2_amd import kv_formats as kvf
from oracle import kv_oracle as oracle

pytestmark = pytest.mark.gpu

INT_VIEW = {torch.float16: torch.int16, torch.bfloat16: torch.int16, torch.float32: torch.int32,
            torch.int64: torch.int64, torch.uint8: torch.uint8}


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(INT_VIEW[t.dtype]).numpy()


def rand(shape, dtype, seed, device):
    g = torch.Generator(device=device).manual_seed(seed)
    return torch.randn(shape, generator=g, device=device).to(dtype)


# --------------------------------------------------------------- flat packet ---

def test_flat_concat_reference_example_and_views(device):
    # kv_cache_communication.py:75-81: 32 layers of [1, 150, 2, 32, 128] fp16
    layers = {i: rand((1, 150, 2, 32, 128), torch.float16, i, device) for i in range(32)}
    print("flat_concat 32 x [1,150,2,32,128] fp16", flush=True)
    flat = kvf.flat_concat(list(layers.values()))
    np.testing.assert_array_equal(bits(flat), oracle.flat_concat([bits(t) for t in layers.values()]))
    views = kvf.flat_views(flat, [t.shape for t in layers.values()])
    for i, t in layers.items():
        assert torch.equal(views[i], t)


@pytest.mark.parametrize("case", ["strided", "transposed", "odd", "wide", "many", "empty"])
def test_flat_concat_layouts(device, case):
    print(f"flat_concat layout {case}", flush=True)
    if case == "strided":  # cache views [B, L, 2, Hkv, D] of [B, S, ...] (batch-strided rows)
        big = rand((3, 4, 40, 2, 8, 128), torch.bfloat16, 1, device)
        tensors = [big[l, :, :33] for l in range(3)]
    elif case == "transposed":  # no block description: made contiguous first
        tensors = [rand((6, 5, 4), torch.float32, 2, device).permute(2, 0, 1)]
    elif case == "odd":  # 105 fp16 elements: 2-byte vectors; 4-byte offset in the packet
        tensors = [rand((3, 5, 7), torch.float16, 3, device), rand((2, 2), torch.float16, 4, device)]
    elif case == "wide":  # one row of 16 MiB: split across many tiles
        tensors = [rand((1, 4096, 2, 8, 128), torch.bfloat16, 5, device)]
    elif case == "many":  # 40 layers > 32 spans per launch
        tensors = [rand((1, 9, 2, 1, 16), torch.float32, 6 + i, device) for i in range(40)]
    else:  # empty tensors among full ones
        tensors = [rand((0, 4), torch.float16, 7, device), rand((2, 4), torch.float16, 8, device),
                   rand((3, 0), torch.float16, 9, device)]
    flat = kvf.flat_concat(tensors)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(flat), oracle.flat_concat([bits(t) for t in tensors]))


def _wire_worker(rank, rendezvous):
    torch.cuda.set_device(0)
    dist.init_process_group("gloo", rank=rank, world_size=2, init_method=Path(rendezvous).as_uri(),
                            timeout=timedelta(seconds=60))
    try:
        dev = torch.device("cuda", 0)
        g = torch.Generator(device="cuda").manual_seed(11)
        big = torch.randn((2, 3, 24, 2, 4, 64), generator=g, device="cuda").to(torch.float16)
        kv = {i: big[i % 2, :1, :17] for i in range(6)}  # [1, 17, 2, 4, 64] views of a longer cache
        logits = torch.randn((2, 320), generator=g, device="cuda").to(torch.float16)
        if rank == 0:
            kvf.kv_cache_communication_send(logits, 17, kv, dst=1)
        else:
            got_logits, seqlen_og, got_kv = kvf.kv_cache_communication_recv(src=0, device=dev)
            assert seqlen_og == 17 and got_logits.is_cuda and torch.equal(got_logits, logits)
            assert list(got_kv) == list(range(6))
            for i in range(6):
                assert got_kv[i].shape == (1, 17, 2, 4, 64) and got_kv[i].is_cuda
                assert torch.equal(got_kv[i].view(torch.int16), kv[i].view(torch.int16)), i
            # the layers are consecutive views of one received buffer
            assert got_kv[1].data_ptr() - got_kv[0].data_ptr() == 17 * 2 * 4 * 64 * 2
        dist.barrier()
    finally:
        dist.destroy_process_group()


def test_flat_packet_wire_between_two_processes(tmp_path):
    print("legacy flat packet over gloo, 2 processes", flush=True)
    mp.spawn(_wire_worker, args=(str(tmp_path / "rendezvous"),), nprocs=2, join=True)


# --------------------------------------------------------- zero-pad batching ---

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_batch_reference_example(device, dtype):
    # kv_cache_batch.py:118-126: [1, 150, ...] and [1, 128, ...] (32 heads -> 4
    # here), logits [1, V] and [3, V]
    print(f"batch_pad reference example {dtype}", flush=True)
    dicts = [{i: rand((1, 150, 2, 4, 128), dtype, 20 + i, device) for i in range(4)},
             {i: rand((1, 128, 2, 4, 128), dtype, 40 + i, device) for i in range(4)}]
    logits = [rand((1, 320), dtype, 1, device), rand((3, 320), dtype, 2, device)]
    got_logits, got = kvf.batch_logits_and_key_value_memory_dict(logits, dicts)
    assert got_logits.shape == (4, 320)
    np.testing.assert_array_equal(bits(got_logits), np.concatenate([bits(l) for l in logits]))
    for key in range(4):
        assert got[key].shape == (2, 150, 2, 4, 128)
        np.testing.assert_array_equal(bits(got[key]), oracle.batch_pad([bits(d[key]) for d in dicts]))
    assert kvf.batched_lengths(dicts) == [150, 128]


def test_batch_pad_ragged_strided_and_empty(device):
    print("batch_pad ragged / strided / empty requests", flush=True)
    caches = rand((3, 5, 64, 2, 8, 128), torch.bfloat16, 3, device)  # [layer, B, S, ...]
    lens = [(2, 61), (1, 7), (0, 5), (2, 0), (1, 64)]  # (sequences, positions) per request
    dicts, b0 = [], 0
    for b, s in lens:
        dicts.append({l: caches[l, b0 % 5:b0 % 5 + b, :s] for l in range(3)})  # batch-strided views
        b0 += 1
    _, got = kvf.batch_logits_and_key_value_memory_dict([torch.zeros((1, 4), device=device)] * len(lens), dicts)
    for l in range(3):
        np.testing.assert_array_equal(bits(got[l]), oracle.batch_pad([bits(d[l]) for d in dicts]))
    assert kvf.batched_lengths(dicts) == [61, 61, 7, 0, 0, 64]


def test_batch_pad_sizes_differing_between_layers(device):
    # each key is padded to its own longest request, as the reference does
    print("batch_pad per-key lengths", flush=True)
    dicts = [{0: rand((1, 9, 2, 2, 16), torch.float16, 1, device), 1: rand((1, 4, 2, 2, 16), torch.float16, 2, device)},
             {0: rand((2, 3, 2, 2, 16), torch.float16, 3, device), 1: rand((2, 11, 2, 2, 16), torch.float16, 4, device)}]
    got = kvf.batch_key_value_memory_dicts(dicts)
    for key, rows in ((0, 9), (1, 11)):
        assert got[key].shape == (3, rows, 2, 2, 16)
        np.testing.assert_array_equal(bits(got[key]), oracle.batch_pad([bits(d[key]) for d in dicts]))


def test_batch_pad_four_byte_rows_and_many_spans(device):
    # 12-byte rows (fp16, 2 x 1 x 3) -> 4-byte vectors; 20 layers x 3 requests
    # x 2 spans > 32 spans per launch
    print("batch_pad 12-byte rows, 120 spans", flush=True)
    dicts = [{l: rand((b, s, 2, 1, 3), torch.float16, 100 * l + b, device) for l in range(20)}
             for b, s in ((1, 9), (2, 4), (1, 1))]
    got = kvf.batch_key_value_memory_dicts(dicts)
    for l in range(20):
        np.testing.assert_array_equal(bits(got[l]), oracle.batch_pad([bits(d[l]) for d in dicts]))
    # an explicit longer padding (room for decode appends)
    got = kvf.batch_key_value_memory_dicts(dicts, max_rows=16)
    np.testing.assert_array_equal(bits(got[3]), oracle.batch_pad([bits(d[3]) for d in dicts], max_rows=16))
    with pytest.raises(ValueError):
        kvf.batch_key_value_memory_dicts(dicts, max_rows=8)


# ------------------------------------------------------------ TP head concat ---

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_head_concat_tp8_to_tp1(device, dtype):
    # Llama-2-70B: 8 KV heads over TP 8 -> one [B, S, 2, 8, 128] cache per layer
    print(f"head_concat TP-8 shards {dtype}", flush=True)
    shards = [{l: rand((4, 300, 2, 1, 128), dtype, 10 * j + l, device) for l in range(3)} for j in range(8)]
    logits, seqlen, got = kvf.tensor_parallel_dim_concat([torch.ones(2, device=device)] * 8, [300] * 8, shards)
    assert seqlen == 300 and torch.equal(logits, torch.ones(2, device=device))
    for l in range(3):
        assert got[l].shape == (4, 300, 2, 8, 128)
        np.testing.assert_array_equal(bits(got[l]), oracle.concat_dim([bits(d[l]) for d in shards]))


def test_head_concat_uneven_strided_and_empty_shards(device):
    print("head_concat uneven / strided / empty shards", flush=True)
    big = rand((2, 3, 50, 2, 3, 64), torch.float16, 5, device)  # [layer, B, S, 2, 3, D]
    shards = [{l: big[l, :, :41, :, :1] for l in range(2)},      # strided in S and heads
              {l: big[l, :, :41] for l in range(2)},             # 3 heads, batch-strided
              {l: torch.empty((3, 41, 2, 0, 64), dtype=torch.float16, device=device) for l in range(2)},
              {l: rand((3, 41, 2, 2, 64), torch.float16, 60 + l, device) for l in range(2)}]
    got = kvf.concat_dicts(shards)
    for l in range(2):
        assert got[l].shape == (3, 41, 2, 6, 64)
        np.testing.assert_array_equal(bits(got[l]), oracle.concat_dim([bits(d[l]) for d in shards]))


@pytest.mark.parametrize("dim", [-2, 1, 4, 0])
def test_concat_dicts_other_dims(device, dim):
    print(f"concat_dicts dim={dim}", flush=True)
    shards = []
    for j, n in enumerate((2, 1, 3)):
        shape = [3, 5, 2, 2, 16]
        shape[dim % 5] = n
        shards.append({l: rand(tuple(shape), torch.float32, 7 * j + l, device) for l in range(2)})
    got = kvf.concat_dicts(shards, dim=dim)
    for l in range(2):
        np.testing.assert_array_equal(bits(got[l]), oracle.concat_dim([bits(d[l]) for d in shards], dim))


def test_head_concat_many_layers_split_launches(device):
    # 40 layers x 8 shards = 320 spans; 64-byte rows (fp32, D 16)
    print("head_concat 320 spans", flush=True)
    shards = [{l: rand((2, 7, 2, 1, 16), torch.float32, 1000 * j + l, device) for l in range(40)}
              for j in range(8)]
    got = kvf.concat_dicts(shards)
    for l in (0, 31, 32, 39):
        np.testing.assert_array_equal(bits(got[l]), oracle.concat_dim([bits(d[l]) for d in shards]))


def test_formats_reject_host_tensors_and_mismatches(device):
    with pytest.raises(ValueError, match="no CPU fallback"):
        kvf.flat_concat([torch.zeros(3)])
    a = torch.zeros((1, 4, 2, 1, 8), device=device)
    with pytest.raises(ValueError):
        kvf.flat_concat([a, a.half()])
    with pytest.raises(ValueError):
        kvf.batch_key_value_memory_dicts([{0: a}, {0: torch.zeros((1, 4, 2, 2, 8), device=device)}])
    with pytest.raises(ValueError):
        kvf.concat_dicts([{0: a}, {0: torch.zeros((1, 5, 2, 1, 8), device=device)}])
