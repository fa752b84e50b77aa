"""The graph-captured decode step (ops.DecodeStepGraph) against eager calls.

Every replay is compared with the eager fused append+attend of the same
step (same kernels and partitions, so bit-exact), with fresh q/kv_new
written in place and eager work plus synchronisation between replays; one
step is also checked against the float64 oracle.  The work-list graphs (one
per step, lists planned up front) are compared the same way with the eager
work-list calls; planning a list under capture is refused."""
import numpy as np
import pytest
import torch

from hexgen2_amd import _lib, ops
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


KERNEL_NAMES = {v: k for k, v in _lib.KERNELS.items()}


@pytest.mark.parametrize("hq,hkv,d,dtype,kernel,partition,single", [
    (32, 8, 128, torch.bfloat16, "valu", 64, True),
    (32, 8, 128, torch.bfloat16, "mfma", 128, True),
    (32, 8, 128, torch.bfloat16, "valu", 64, False),
    (8, 1, 128, torch.bfloat16, "auto", 0, True),
    (32, 4, 64, torch.float16, "auto", 0, True),
    (32, 4, 64, torch.float16, "auto", 64, False),
    (4, 4, 16, torch.float32, "auto", 64, True),
    (32, 8, 128, torch.bfloat16, "rows", 32, True),
    (32, 32, 128, torch.float16, "rows", 0, True)])
def test_graph_work_list_replays_match_eager_lists(device, hq, hkv, d, dtype, kernel, partition, single):
    """DecodeStepGraph(lens=...): every step's work list is planned up front
    (StepWorkLists) and captured in a graph of its own, and the last layer's
    kernel stores the new lengths to ``positions``; each replay equals, bit
    for bit, the eager work-list calls of the same step with the same chunk
    (merged in the attention kernel, or by the second kernel), with fresh q
    and kv_new written in place and eager work between the replays.  Rows
    cross chunk boundaries during the replays, so item and partition counts
    change from graph to graph."""
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

    def eager_step(chunk, step_kernel):
        for l in range(layers):
            ops.decode_attention(q[l], cache_e[l], max_seqlen=max_seqlen, seqlens=pos_e, kv_new=kv_new[l],
                                 out=out_e[l], kernel=step_kernel, lens=host, partition=chunk,
                                 single_launch=single)
        pos_e.add_(1)
        host[:] = [n + 1 for n in host]

    def refill():
        q.copy_(torch.randn(q.shape, generator=g, device=device).to(dtype))
        kv_new.copy_(torch.randn(kv_new.shape, generator=g, device=device).to(dtype))

    ops.device_status()  # start clear
    refill()
    eager_step(partition, kernel)  # also loads the kernels before capture
    cache_g.copy_(cache_e)
    pos_g = pos_e.clone()
    torch.cuda.synchronize()
    graph = ops.DecodeStepGraph(q, cache_g, out_g, kv_new, pos_g, max_seqlen, kernel=kernel, lens=host,
                                partition=partition, single_launch=single)
    lists = graph.lists
    assert len(lists) == steps - 1 and (lists.xcds > 0) == single
    if partition:
        assert set(lists.chunks) == {partition}
    if kernel != "auto":
        assert set(lists.kernels) == {_lib.KERNELS[kernel]}
    counts = []
    for step in range(steps - 1):
        refill()
        eager_step(lists.chunks[step], KERNEL_NAMES[lists.kernels[step]])  # as the step was planned
        graph.replay()
        torch.cuda.synchronize()
        counts.append(int(lists[step].parts.sum()))  # partitions over all segments
        assert torch.equal(pos_g, pos_e), f"step {step}: positions differ"
        assert torch.equal(cache_g, cache_e), f"step {step}: cache differs"
        assert torch.equal(out_g, out_e), f"step {step}: output differs"
    if partition:
        assert counts[0] < counts[-1], "a row crossed a chunk boundary during the replays"
    status = ops.device_status()
    print(f"  device status {status:#x}", flush=True)
    assert status & _lib.STATUS_ERRORS == 0
    with pytest.raises(RuntimeError, match="replays"):
        graph.replay()  # past the last length max_seqlen allows
    graph.restart()
    assert graph.step == 0


def test_work_list_graphs_replayed_on_a_side_stream(device):
    """Work-list step graphs captured and replayed on a stream of the
    caller's (whose queue may start dispatching at another XCD than the
    default stream's) equal the eager calls on the default stream, bit for
    bit, with the row-block kernel the library picks for a large call."""
    layers, lens, steps = 2, [3000, 40, 2500, 4029, 2800, 4000, 12, 3900], 3  # 83 MB per call
    hq, hkv, d, dtype = 32, 8, 128, torch.bfloat16
    cap = max(lens) + steps + 3
    max_seqlen = max(lens) + steps
    g = torch.Generator(device=device).manual_seed(24)
    cache_e = torch.randn((layers, len(lens), cap, 2, hkv, d), generator=g, device=device).to(dtype)
    cache_g = cache_e.clone()
    q = torch.randn((layers, len(lens), 1, hq, d), generator=g, device=device).to(dtype)
    kv_new = torch.randn((layers, len(lens), 2, hkv, d), generator=g, device=device).to(dtype)
    out_e = torch.empty((layers, len(lens), 1, hq, d), dtype=dtype, device=device)
    out_g = torch.empty_like(out_e)
    pos_e = torch.tensor(lens, dtype=torch.int32, device=device)
    pos_g = pos_e.clone()
    host = list(lens)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for l in range(layers):  # loads the kernels before capture (on scratch copies)
            ops.decode_attention(q[l], cache_e[l].clone(), max_seqlen=max_seqlen, seqlens=pos_e, kv_new=kv_new[l],
                                 lens=host)
        graph = ops.DecodeStepGraph(q, cache_g, out_g, kv_new, pos_g, max_seqlen, lens=host)
    torch.cuda.synchronize()
    lists = graph.lists
    names = {v: k for k, v in _lib.KERNELS.items()}
    assert lists.xcds > 0 and set(lists.kernels) == {_lib.KERNELS["rows"]}
    for step in range(steps - 1):
        for l in range(layers):
            ops.decode_attention(q[l], cache_e[l], max_seqlen=max_seqlen, seqlens=pos_e, kv_new=kv_new[l],
                                 out=out_e[l], lens=host, partition=lists.chunks[step],
                                 kernel=names[lists.kernels[step]])
        pos_e.add_(1)
        host = [n + 1 for n in host]
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(pos_g, pos_e), f"step {step}: positions differ"
        assert torch.equal(cache_g.view(torch.int16), cache_e.view(torch.int16)), f"step {step}: caches differ"
        assert torch.equal(out_g, out_e), f"step {step}: outputs differ"
    assert ops.device_status() & _lib.STATUS_ERRORS == 0


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")  # the refused capture records nothing
def test_planning_under_capture_is_refused(device):
    """A work list planned inside graph capture would record a copy from a
    temporary host buffer: decode_attention(lens=...) and AttendPlan(lens=...)
    raise ValueError there, and leave the stream usable."""
    q = torch.randn((2, 1, 8, 64), device=device).to(torch.float16)
    cache = torch.randn((2, 64, 2, 2, 64), device=device).to(torch.float16)
    out = torch.empty_like(q)
    seqlens = torch.tensor([10, 20], dtype=torch.int32, device=device)
    ops.decode_attention(q, cache, max_seqlen=21, seqlens=seqlens, out=out, lens=[10, 20])  # loads the kernel
    torch.cuda.synchronize()
    plan = ops.AttendPlan(q, cache, out, max_seqlens=[21], seqlens=seqlens, lens=[10, 20])
    for call in (lambda: ops.decode_attention(q, cache, max_seqlen=21, seqlens=seqlens, out=out, lens=[10, 20]),
                 lambda: plan(q, cache, out, None, 0, 21)):
        graph = torch.cuda.CUDAGraph()
        with pytest.raises(ValueError, match="graph capture"):
            with torch.cuda.graph(graph):
                call()
        torch.cuda.synchronize()
    ops.decode_attention(q, cache, max_seqlen=21, seqlens=seqlens, out=out, lens=[10, 20])
    torch.cuda.synchronize()


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
