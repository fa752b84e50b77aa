"""The CPU baselines time oracle/cpu_path.py, the reference's own torch
operations restated on host tensors.  Those timings compare like with like
only if the operations compute what the path computes: each one is checked
here against the numpy oracle on small seeded inputs (bit-exact for the byte
moves, fp64-close for attention)."""
import numpy as np
import pytest
import torch

from oracle import cpu_path, kv_oracle as oracle


def _rand(shape, seed, dtype=torch.float32):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed)).to(dtype)


def test_pack_unpack_append_are_the_oracle_moves():
    lens, cap = [5, 1, 7], 9
    layers = [_rand((3, cap, 2, 2, 4), l) for l in range(2)]
    packed = cpu_path.pack(layers, lens)
    want = oracle.pack([t.numpy() for t in layers], lens)
    for l in range(2):
        np.testing.assert_array_equal(packed[l].numpy(), want[l])
    full = cpu_path.unpack(packed, cap, lens)
    for l in range(2):
        for b, n in enumerate(lens):
            np.testing.assert_array_equal(full[l][b, :n].numpy(), layers[l][b, :n].numpy())
    kv = _rand((3, 2, 2, 4), 9)
    cache = layers[0].clone()
    cpu_path.append(cache, kv, [5, 1, 8])
    np.testing.assert_array_equal(cache.numpy(), oracle.append(layers[0].numpy(), kv.numpy(), [5, 1, 8]))


@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 2)])
def test_attend_is_the_oracle_attention(hq, hkv):
    lens = [6, 1, 11]
    q = _rand((3, 1, hq, 16), 1)
    cache = _rand((3, 12, 2, hkv, 16), 2)
    got = cpu_path.attend(q, cache, lens).double().numpy()
    want = oracle.attend(q.double().numpy(), cache.double().numpy(), lens)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-6)


def test_format_ops_are_the_oracle_formats():
    big = _rand((2, 3, 10, 2, 4, 8), 3, torch.float16)
    tensors = [big[0, :, :7], big[1, 1:3], big[0, :, :, :, 1:3]]
    np.testing.assert_array_equal(cpu_path.flat_concat(tensors).numpy(),
                                  oracle.flat_concat([t.numpy() for t in tensors]))
    dicts = [{l: big[l, i:i + 1, :n] for l in range(2)} for i, n in enumerate([4, 10, 1])]
    got = cpu_path.batch_pad(dicts)
    for l in range(2):
        np.testing.assert_array_equal(got[l].numpy(), oracle.batch_pad([d[l].numpy() for d in dicts]))
    shards = [{l: big[l, :, :, :, h:h + 1] for l in range(2)} for h in range(4)]
    got = cpu_path.concat_dicts(shards)
    for l in range(2):
        np.testing.assert_array_equal(got[l].numpy(), oracle.concat_dim([s[l].numpy() for s in shards]))


@pytest.mark.parametrize("dtype,pack", [(torch.float16, 8), (torch.float32, 4)])
def test_ft_store_is_the_oracle_layout(dtype, pack):
    kv = _rand((2, 5, 2, 3, 16), 4, dtype)
    cap = 7
    k_cache = torch.full((2, 3, 16 // pack, cap, pack), -3.0, dtype=dtype)
    v_cache = torch.full((2, 3, cap, 16), -3.0, dtype=dtype)
    cpu_path.ft_store(kv, k_cache, v_cache)
    k_ref, v_ref = oracle.ft_layout(kv.numpy(), pack)
    np.testing.assert_array_equal(k_cache[:, :, :, :5].numpy(), k_ref)
    np.testing.assert_array_equal(v_cache[:, :, :5].numpy(), v_ref)
    assert (k_cache[:, :, :, 5:] == -3).all() and (v_cache[:, :, 5:] == -3).all()
