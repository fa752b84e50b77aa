"""The full-size attention parity tests can see a misread chunk.

tests/test_gpu_scale.py compares the HIP attention with the oracle within
8e-3 (bf16).  Here, on the CPU, the oracle itself is given one wrong
1280-position chunk (the work-list chunk at Llama-3-8B's size) and its
output must move by well over that tolerance.  In rows of Llama-3-8B's
length (8448 positions) it does at the keys' own scale; in the long-context
test's rows (10^5 positions) the weight of a row spreads over so many keys
that the same mistake can stay within the tolerance, which is why that test
draws its queries at three times the keys' scale (and the full-size tests at
twice, for margin)."""
import numpy as np
import torch

from oracle import kv_oracle as oracle

TOL_BF16 = 8e-3


def bf16(shape, gen, scale=1.0):
    return (scale * torch.randn(shape, generator=gen)).to(torch.bfloat16).double().numpy()


def misread_shift(n, q_scale, kv_heads, q_heads, chunk=1280, seed=0):
    """max |attention with one chunk of keys/values replaced - attention| over
    one row of n positions (head_dim 128)."""
    g = torch.Generator().manual_seed(seed)
    q = bf16((1, 1, q_heads, 128), g, q_scale)
    cache = bf16((1, n, 2, kv_heads, 128), g)
    other = cache.copy()
    start = (n // chunk // 2) * chunk
    other[0, start:start + chunk] = bf16((chunk, 2, kv_heads, 128), g)
    return float(np.abs(oracle.attend(q, cache, [n]) - oracle.attend(q, other, [n])).max())


# One KV head of 4 query heads (Llama-3-8B's group) keeps the host arrays
# small; a row's statistics do not depend on how many heads there are.

def test_full_size_rows_expose_a_misread_chunk():
    # Llama-3-8B's longest rows; unit and doubled query scale
    for scale in (1.0, 2.0):
        for seed in range(2):
            assert misread_shift(8448, scale, 1, 4, seed=seed) > 3 * TOL_BF16


def test_long_context_rows_need_scaled_queries():
    unit = [misread_shift(70001, 1.0, 1, 4, seed=s) for s in range(2)]
    scaled = [misread_shift(70001, 3.0, 1, 4, seed=s) for s in range(2)]
    assert min(unit) < TOL_BF16, unit
    assert min(scaled) > 3 * TOL_BF16, scaled
