"""The graph-captured decode step (ops.DecodeStepGraph) against eager calls.

Every replay is compared with the eager fused append+attend of the same
step (same kernels and partitions, so bit-exact), with fresh q/kv_new
written in place and eager work plus synchronisation between replays; one
step is also checked against the float64 oracle.  The work-list graph is
compared the same way with the eager work-list calls."""
import numpy as np
import pytest
import torch

from hexgen2_amd import ops
from oracle import kv_oracle as oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("hq,hkv,d,dtype,kernel", [(32, 8, 128, torch.bfloat16, "valu"),
                                                   (32, 8, 128, torch.bfloat16, "mfma"),
                                                   (32, 4, 64, torch.float16, "auto"),
                                                   (4, 4, 16, torch.float32, "auto")])
def test_graph_replays_match_eager_steps(device, hq, hkv, d, dtype, kernel):
    layers, lens, steps = 3, [1, 40, 300, 1029, 7], 5
    cap = max(lens) + steps + 3
    max_seqlen = max(lens) + steps
    g = torch.Generator(device=device).manual_seed(21)
    cache_e = torch.randn((layers, len(lens), cap, 2, hkv, d), generator=g, device=device).to(dtype)
    cache_g = cache_e.clone()
    q = torch.empty((layers, len(lens), 1, hq, d), dtype=dtype, device=device)
    kv_new = torch.empty((layers, len(lens), 2, hkv, d), dtype=dtype, device=device)
    out_e = torch.empty((layers, len(lens), 1, hq, d), dtype=dtype, device=device)
    out_g = torch.empty_like(out_e)
    pos_e = torch.tensor(lens, dtype=torch.int32, device=device)
    pos_g = pos_e.clone()

    def eager_step():
        for l in range(layers):
            ops.decode_attention(q[l], cache_e[l], max_seqlen=max_seqlen, seqlens=pos_e, kv_new=kv_new[l],
                                 out=out_e[l], kernel=kernel)
        pos_e.add_(1)

    q.copy_(torch.randn(q.shape, generator=g, device=device).to(dtype))
    kv_new.copy_(torch.randn(kv_new.shape, generator=g, device=device).to(dtype))
    eager_step()  # also loads the kernels before capture
    cache_g.copy_(cache_e)
    pos_g.copy_(pos_e)
    torch.cuda.synchronize()
    graph = ops.DecodeStepGraph(q, cache_g, out_g, kv_new, pos_g, max_seqlen, kernel=kernel)
    for step in range(steps - 1):
        q.copy_(torch.randn(q.shape, generator=g, device=device).to(dtype))
        kv_new.copy_(torch.randn(kv_new.shape, generator=g, device=device).to(dtype))
        before = cache_e[0].clone()
        eager_step()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(pos_g, pos_e)
        assert torch.equal(cache_g, cache_e), f"step {step}: cache differs"
        assert torch.equal(out_g, out_e), f"step {step}: output differs"
        if step == 1:
            attended = pos_e.tolist()  # keys attended by this step = lengths after its append
            ref = oracle.attend(q[0].double().cpu().numpy(), cache_e[0].double().cpu().numpy(), attended)
            err = np.abs(out_e[0].double().cpu().numpy() - ref).max()
            assert err <= {torch.float16: 2e-3, torch.bfloat16: 8e-3, torch.float32: 2e-5}[dtype]
            # the step appended exactly one row per sequence
            changed = (cache_e[0] != before).flatten(2).any(-1)
            assert changed.sum() <= len(lens)


@pytest.mark.parametrize("hq,hkv,d,dtype,kernel,partition", [(32, 8, 128, torch.bfloat16, "valu", 64),
                                                             (32, 8, 128, torch.bfloat16, "mfma", 128),
                                                             (8, 1, 128, torch.bfloat16, "auto", 0),
                                                             (32, 4, 64, torch.float16, "auto", 64),
                                                             (4, 4, 16, torch.float32, "auto", 64)])
def test_graph_work_list_replays_match_eager_lists(device, hq, hkv, d, dtype, kernel, partition):
    """DecodeStepGraph(lens=...): each replay uploads its step's work list
    into the buffers the graph captured (padded to the last replay's item
    count) and equals, bit for bit, the eager work-list call of the same
    step with the same chunk; rows cross chunk boundaries during the
    replays, so item and partition counts grow under the fixed capture."""
    # after the eager step, replay k attends lens + k + 2 keys: sequence 2
    # crosses 384 (a multiple of 64 and 128) at k = 1, sequence 4 crosses 64
    layers, lens, steps = 3, [1, 40, 381, 1029, 62], 6
    cap = max(lens) + steps + 3
    max_seqlen = max(lens) + steps
    g = torch.Generator(device=device).manual_seed(23)
    cache_e = torch.randn((layers, len(lens), cap, 2, hkv, d), generator=g, device=device).to(dtype)
    cache_g = cache_e.clone()
    q = torch.empty((layers, len(lens), 1, hq, d), dtype=dtype, device=device)
    kv_new = torch.empty((layers, len(lens), 2, hkv, d), dtype=dtype, device=device)
    out_e = torch.empty((layers, len(lens), 1, hq, d), dtype=dtype, device=device)
    out_g = torch.empty_like(out_e)
    pos_e = torch.tensor(lens, dtype=torch.int32, device=device)
    host = list(lens)

    def eager_step(chunk):
        for l in range(layers):
            ops.decode_attention(q[l], cache_e[l], max_seqlen=max_seqlen, seqlens=pos_e, kv_new=kv_new[l],
                                 out=out_e[l], kernel=kernel, lens=host, partition=chunk)
        pos_e.add_(1)
        host[:] = [n + 1 for n in host]

    def refill():
        q.copy_(torch.randn(q.shape, generator=g, device=device).to(dtype))
        kv_new.copy_(torch.randn(kv_new.shape, generator=g, device=device).to(dtype))

    refill()
    eager_step(partition)  # also loads the kernels before capture
    cache_g.copy_(cache_e)
    pos_g = pos_e.clone()
    torch.cuda.synchronize()
    graph = ops.DecodeStepGraph(q, cache_g, out_g, kv_new, pos_g, max_seqlen, kernel=kernel, lens=host,
                                partition=partition)
    lists = graph.lists
    assert lists.replays == steps - 1
    if partition:
        assert lists.chunk == partition
    counts = []
    for step in range(steps - 1):
        refill()
        eager_step(lists.chunk)
        graph.replay()
        torch.cuda.synchronize()
        counts.append(lists.filled[step % 2])
        assert torch.equal(pos_g, pos_e)
        assert torch.equal(cache_g, cache_e), f"step {step}: cache differs"
        assert torch.equal(out_g, out_e), f"step {step}: output differs"
    assert counts == sorted(counts) and counts[-1] == lists.capacity
    if partition:
        assert counts[0] < counts[-1], "a row crossed a chunk boundary during the replays"
    with pytest.raises(RuntimeError, match="replays"):
        graph.replay()  # past the last length max_seqlen allows


@pytest.mark.parametrize("hq,hkv,d,dtype,rot", [(32, 8, 128, torch.bfloat16, 128),
                                                (8, 1, 64, torch.float16, 32),
                                                (4, 4, 16, torch.float32, 0)])
def test_ft_graph_replays_match_eager_steps(device, hq, hkv, d, dtype, rot):
    """ops.FtDecodeStepGraph: every replay equals the eager ft_attend calls of
    the same step bit for bit (caches, outputs, positions)."""
    layers, lens, steps = 3, [1, 40, 300, 1029, 7], 5
    cap = max(lens) + steps + 3
    max_position = max(lens) + steps
    batch = len(lens)
    g = torch.Generator(device=device).manual_seed(22)
    k_shape, v_shape = ops.ft_cache_shapes(batch, hkv, cap, d, dtype)
    k_e = torch.randn((layers,) + k_shape, generator=g, device=device).to(dtype)
    v_e = torch.randn((layers,) + v_shape, generator=g, device=device).to(dtype)
    k_g, v_g = k_e.clone(), v_e.clone()
    q = torch.empty((layers, batch, hq, d), dtype=dtype, device=device)
    new = torch.empty((layers, 2, batch, hkv, d), dtype=dtype, device=device)
    out_e = torch.empty_like(q)
    out_g = torch.empty_like(q)
    pos_e = torch.tensor(lens, dtype=torch.int32, device=device)
    pos_g = pos_e.clone()

    def eager_step():
        for l in range(layers):
            ops.ft_attend(q[l], new[l, 0], new[l, 1], k_e[l], v_e[l], max_position=max_position, positions=pos_e,
                          rotary_dim=rot, out=out_e[l])
        pos_e.add_(1)

    def refill():
        q.copy_(torch.randn(q.shape, generator=g, device=device).to(dtype))
        new.copy_(torch.randn(new.shape, generator=g, device=device).to(dtype))

    refill()
    eager_step()  # also loads the kernels before capture
    k_g.copy_(k_e)
    v_g.copy_(v_e)
    pos_g.copy_(pos_e)
    torch.cuda.synchronize()
    graph = ops.FtDecodeStepGraph(q, k_g, v_g, out_g, new[:, 0], new[:, 1], pos_g, max_position, rotary_dim=rot)
    for step in range(steps - 1):
        refill()
        eager_step()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(pos_g, pos_e)
        assert torch.equal(k_g, k_e) and torch.equal(v_g, v_e), f"step {step}: caches differ"
        assert torch.equal(out_g, out_e), f"step {step}: output differs"
