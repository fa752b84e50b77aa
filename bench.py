#!/usr/bin/env python3
"""Benchmark of the KV-cache data path on one MI355X.

One bench step is one whole handoff-and-decode job on synthetic data of the
Llama-3-8B shape (32 layers, 8 KV / 32 query heads, head_dim 128, bf16,
batch 64, prompt lengths U[128, 8192] seeded): pack every layer's live rows
into the handoff buffer, unpack them into the decode cache, then 256 decode
steps of fused KV append + single-query GQA attention over all 32 layers,
each step one replay of its own captured HIP graph over its work list
(planned up front with hexkv_attend_plan for the device's XCDs, split rows
merged inside the attention kernel).  Inputs are resident in HBM before the
timed region.

Prints one JSON line: ``value`` = pack+unpack GB/s (algorithmic bytes), with
the decode append+attend time per step, the roofline of the dominant kernel
(decode attention) and the CPU baseline (the reference's PyTorch ops on this
host's cores, on a bounded sample of the same workload).  After the timed
job, outside it: ``workloads`` -- the same measurements (fewer steps) for the
TinyLlama-1.1B, Llama-2-7B and Llama-2-70B TP-8 shapes, each with its own
roofline and CPU baseline -- and ``formats`` (the legacy KV formats) with
their CPU figures.  ``--ft`` adds the FasterTransformer cache layout.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from hexgen2_amd import _lib, ops  # noqa: E402
from hexgen2_amd.workloads import WORKLOADS, workload  # noqa: E402

HBM_PEAK_GBS = 8000.0
METRIC = "KV pack+unpack GB/s (% HBM peak); decode append+attend µs/step at Llama-3-8B"
TRAFFIC_FILE = ROOT / "profiles" / "traffic.json"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Job:
    """Device buffers of one workload and the timed job pass."""

    def __init__(self, w, device, kernel="auto", grid=False, single_launch=True):
        self.w = w
        self.kernel = kernel
        L, B, S = w.layers, w.batch, w.capacity
        shape = (L, B, S, 2, w.kv_heads, w.head_dim)
        g = torch.Generator(device=device).manual_seed(w.seed + 1)
        self.prefill = torch.empty(shape, dtype=w.dtype, device=device)
        for l in range(L):  # K/V ~ N(0, 1)
            self.prefill[l].normal_(generator=g)
        self.packed = torch.empty((L, w.live_rows, 2, w.kv_heads, w.head_dim), dtype=w.dtype, device=device)
        self.decode = torch.empty(shape, dtype=w.dtype, device=device)
        self.decode_layers = list(self.decode.unbind(0))
        self.q = torch.randn((L, B, 1, w.q_heads, w.head_dim), generator=g, device=device).to(w.dtype)
        self.kv_new = torch.randn((L, B, 2, w.kv_heads, w.head_dim), generator=g, device=device).to(w.dtype)
        self.out = torch.empty((B, 1, w.q_heads, w.head_dim), dtype=w.dtype, device=device)
        self.seqlens = torch.tensor(w.lens, dtype=torch.int32, device=device)
        self.max_len = max(w.lens)
        self.grid, self.single_launch = grid, single_launch
        # Eager decode steps: one parameter block for every layer; with work
        # lists (the lengths are known here) every step's list is planned up
        # front, the same lists the captured graphs run.
        self.plan = ops.AttendPlan(self.q[0], self.decode_layers[0], self.out,
                                   max_seqlens=[self.max_len + t + 1 for t in range(w.decode_steps)],
                                   seqlens=self.seqlens, kv_new=self.kv_new[0], kernel=kernel)
        self.lists = None
        if not grid:
            self.lists = ops.StepWorkLists(self.plan.params, w.lens, w.decode_steps, device, single_launch)
            self.plan.reserve(self.lists.lists)
        self.kernel_name = ops.attend_kernel(self.q[0], self.decode_layers[0], kernel)
        if self.lists is not None:
            # the kernel each step's list was planned with (the row-block kernel
            # for "auto" on large calls)
            names = {v: k for k, v in _lib.KERNELS.items()}
            used = sorted({names[k] for k in self.lists.kernels})
            self.kernel_name = "+".join(used)
        self.positions = self.seqlens.clone()
        self.graph = None
        # TinyLlama's 46 MB handoff fits in the 256 MB MALL: a 512 MB fill
        # between timed steps evicts it
        self.mall_flush = None
        if w.pack_unpack_bytes() < (1 << 30):
            self.mall_flush = torch.empty(512 << 20, dtype=torch.uint8, device=device)
        torch.cuda.synchronize()

    @property
    def schedule(self):
        if self.grid:
            return "uniform grid, split rows merged by a second kernel"
        rows = sum(k == _lib.KERNELS["rows"] for k in self.lists.kernels)
        return ("work lists planned per step up front (hexkv_attend_plan)"
                + (f", for {self.lists.xcds} XCDs: split rows merged in the attention kernel (one launch)"
                   if self.lists.xcds else ", split rows merged by a second kernel")
                + (f"; {rows} of {len(self.lists.kernels)} steps on the row-block kernel (items over "
                   "adjacent KV heads of every cache row)" if rows else ""))

    def capture_graph(self):
        """The all-layer decode step as captured HIP graphs (after an eager
        pass): one per step over its work list, or one over the grid."""
        w = self.w
        self.graph = ops.DecodeStepGraph(list(self.q.unbind(0)), self.decode_layers, [self.out] * w.layers,
                                         list(self.kv_new.unbind(0)), self.positions,
                                         self.max_len + w.decode_steps, kernel=self.kernel,
                                         lens=None if self.grid else w.lens, single_launch=self.single_launch)

    def handoff(self, events=None):
        """pack -> unpack, recording (start, packed, unpacked) events."""
        w, ev = self.w, events
        if self.mall_flush is not None:
            self.mall_flush.fill_(1)
        if ev is not None:
            ev[0].record()
        ops.pack_live(self.prefill, w.lens, out=self.packed)
        if ev is not None:
            ev[1].record()
        ops.unpack_live(self.packed, self.decode, w.lens)
        if ev is not None:
            ev[2].record()

    def run_graph(self, events=None):
        """pack -> unpack -> decode steps replayed from the captured graphs;
        records (start, packed, unpacked, decoded) events.  The decode steps
        run back to back with no event between them: an event recorded after
        every replay put a gap of its own between the graphs (about 10 us a
        step on this GPU), which a decode loop does not have."""
        w, ev = self.w, events
        self.handoff(ev)
        self.positions.copy_(self.seqlens)
        self.graph.restart()
        for t in range(w.decode_steps):
            self.graph.replay()
        if ev is not None:
            ev[3].record()

    def eager_step(self, t):
        """Decode step t launched layer by layer from the host."""
        w = self.w
        if self.lists is not None:
            self.plan.fix_work_list(self.lists[t])
        for l in range(w.layers):
            self.plan(self.q[l], self.decode_layers[l], self.out, self.kv_new[l], t, self.max_len + t + 1)

    def run(self, events=None):
        """pack -> unpack -> decode steps launched eagerly, layer by layer;
        records (start, packed, unpacked, decoded) events."""
        w, ev = self.w, events
        self.handoff(ev)
        for t in range(w.decode_steps):
            self.eager_step(t)
        if ev is not None:
            ev[3].record()

    def decode_mall_busted(self):
        """Average µs of one graph-replayed decode step when the MALL is
        evicted before every step (the fill outside the timed step)."""
        w = self.w
        self.handoff()
        self.positions.copy_(self.seqlens)
        self.graph.restart()
        total = 0.0
        for t in range(w.decode_steps):
            self.mall_flush.fill_(1)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            self.graph.replay()
            e1.record()
            e1.synchronize()
            total += e0.elapsed_time(e1)
        return total * 1e3 / w.decode_steps  # (each step between its own events)

    def traffic_probe(self):
        """A short fixed dispatch sequence for hardware-counter runs
        (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE), in this order:

        1. calibration: the pack kernel on one contiguous 2 GiB sequence, which
           is a plain copy of exactly 2 GiB read + 2 GiB written;
        2. pack of the workload; 3. unpack of the workload;
        4. decode step 0 over every layer (fused append + attend);
        then (formats_traffic_probe, after the job's buffers are freed) one
        call of each legacy format.
        """
        w = self.w
        rows = (2 << 30) // w.row_bytes
        src = torch.ones((1, rows, 2, w.kv_heads, w.head_dim), dtype=w.dtype, device=self.q.device)
        dst = torch.empty((1, rows, 2, w.kv_heads, w.head_dim), dtype=w.dtype, device=self.q.device)
        torch.cuda.synchronize()
        log(f"calibration copy: {rows * w.row_bytes} bytes")
        ops.pack_live([src], [rows], out=[dst[0]])
        torch.cuda.synchronize()
        del src, dst
        log("pack, unpack, one decode step")
        ops.pack_live(self.prefill, w.lens, out=self.packed)
        ops.unpack_live(self.packed, self.decode, w.lens)
        self.eager_step(0)
        torch.cuda.synchronize()
        log("probe done")

    @staticmethod
    def formats_traffic_probe(device):
        """5. one call of each legacy format, in format_cases order."""
        cases = format_cases(device)
        torch.cuda.synchronize()
        for name, run, nbytes, launches, _ in cases:
            log(f"format {name}: {launches} launches, {nbytes} algorithmic bytes")
            run()
        torch.cuda.synchronize()

    def verify(self):
        """Size-independent self-check on the full workload: the unpacked live
        rows equal the prefill cache's (before any append) and the packed
        buffer is the concatenation of live rows; checked on the device."""
        w = self.w
        ops.pack_live(self.prefill, w.lens, out=self.packed)
        ops.unpack_live(self.packed, self.decode, w.lens)
        start = 0
        for b, n in enumerate(w.lens):
            a = self.prefill[:, b, :n]
            if not torch.equal(a, self.decode[:, b, :n]) or not torch.equal(a, self.packed[:, start:start + n]):
                raise AssertionError(f"pack/unpack round trip differs for sequence {b}")
            start += n


def format_cases(device):
    """The legacy KV formats (hexgen2_amd.kv_formats) on Llama-shaped
    synthetic data, as (name, run, algorithmic bytes, launches, extra):
    algorithmic bytes = bytes read + bytes written, zero padding included.

    * flat_packet: 32 layers of one request's live [1, 8192, 2, 8, 128] bf16
      slice of an 8448-position cache, flattened and concatenated;
    * zero_pad_batch: 8 requests of lengths U[128, 4096] (seed 0), 32 layers
      of [1, L_i, 2, 8, 128] bf16, padded to the longest and stacked;
    * tp_head_concat: 16 layers of 8 tensor-parallel shards [8, 4096, 2, 1,
      128] bf16 (Llama-2-70B's KV heads over TP 8) joined into one
      [8, 4096, 2, 8, 128] cache per layer.
    """
    from hexgen2_amd import kv_formats as kvf

    g = torch.Generator(device=device).manual_seed(3)
    row = 2 * 8 * 128 * 2
    # Each case's layers are views of one stacked allocation, so the span
    # engine folds them into one layer dimension: one launch per call.
    cases = []
    cache = torch.empty((32, 1, 8448, 2, 8, 128), dtype=torch.bfloat16, device=device).normal_(generator=g)
    layers = [cache[l, :, :8192] for l in range(32)]
    flat = torch.empty(32 * 8192 * row // 2, dtype=torch.bfloat16, device=device)
    cases.append(("flat_packet", lambda: kvf.flat_concat(layers, out=flat), 2 * 32 * 8192 * row, 1, {}))

    lens = [int(x) for x in torch.randint(128, 4097, (8,), generator=torch.Generator().manual_seed(0))]
    bcache = torch.empty((32, 8, 4096, 2, 8, 128), dtype=torch.bfloat16, device=device).normal_(generator=g)
    dicts = [{l: bcache[l, i:i + 1, :n] for l in range(32)} for i, n in enumerate(lens)]
    cases.append(("zero_pad_batch", lambda: kvf.batch_key_value_memory_dicts(dicts),
                  32 * row * (sum(lens) + 8 * max(lens)), 1, {"lens": lens}))

    shards_t = torch.empty((8, 16, 8, 4096, 2, 1, 128), dtype=torch.bfloat16, device=device).normal_(generator=g)
    shards = [{l: shards_t[j, l] for l in range(16)} for j in range(8)]
    cases.append(("tp_head_concat", lambda: kvf.concat_dicts(shards), 2 * shards_t.numel() * 2, 1, {}))
    return cases


def measure_formats(device, reps=5):
    """Secondary figures, outside the timed steps: GB/s of algorithmic bytes
    of each legacy format (``format_cases``), HIP events over ``reps`` calls."""
    out = {}
    for name, run, nbytes, launches, extra in format_cases(device):
        run()
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ev[0].record()
        for _ in range(reps):
            run()
        ev[1].record()
        torch.cuda.synchronize()
        ms = ev[0].elapsed_time(ev[1]) / reps
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "ms": round(ms, 4),
                     "bytes": int(nbytes), "launches": launches, **extra}
    torch.cuda.empty_cache()
    return out


def measure_ft(device, steps=16):
    """Secondary figures for the FasterTransformer-layout path on one
    Llama-3-8B-shaped layer, outside the timed steps: hexkv_ft_store of a
    64 x 4096-position prefill (GB/s of bytes read + written) and
    ``steps`` hexkv_ft_attend decode steps with full-width rotary over the
    workload's ragged lengths (µs per call; GB/s with the byte accounting of
    hexkv_attend)."""
    w = workload("llama3-8b")
    B, H, Hq, D, dtype = w.batch, w.kv_heads, w.q_heads, w.head_dim, w.dtype
    g = torch.Generator(device=device).manual_seed(w.seed + 7)
    k_shape, v_shape = ops.ft_cache_shapes(B, H, w.capacity, D, dtype)
    k_cache = torch.empty(k_shape, dtype=dtype, device=device).normal_(generator=g)
    v_cache = torch.empty(v_shape, dtype=dtype, device=device).normal_(generator=g)
    out = {}
    kv = torch.randn((B, 4096, 2, H, D), generator=g, device=device).to(dtype)
    ops.ft_store(kv, k_cache, v_cache)
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ev[0].record()
    for _ in range(5):
        ops.ft_store(kv, k_cache, v_cache)
    ev[1].record()
    torch.cuda.synchronize()
    ms = ev[0].elapsed_time(ev[1]) / 5
    nbytes = 2 * kv.numel() * kv.element_size()
    out["ft_store"] = {"gbs": round(nbytes / (ms * 1e-3) / 1e9, 1), "ms": round(ms, 4), "bytes": nbytes,
                       "shape": list(kv.shape)}
    del kv
    q = torch.randn((B, Hq, D), generator=g, device=device).to(dtype)
    new = torch.randn((B, 2, H, D), generator=g, device=device).to(dtype)
    lens = torch.tensor(w.lens, dtype=torch.int32, device=device)
    max_len = max(w.lens)
    ws = torch.empty(max(ops.ft_attend_workspace_bytes(q, k_cache, v_cache, max_len + steps), 16),
                     dtype=torch.uint8, device=device)
    res = torch.empty_like(q)

    def step(t):
        ops.ft_attend(q, new[:, 0], new[:, 1], k_cache, v_cache, max_position=max_len + t, positions=lens,
                      position_bias=t, rotary_dim=D, out=res, workspace=ws)
    step(0)
    torch.cuda.synchronize()
    ev[0].record()
    for t in range(steps):
        step(t)
    ev[1].record()
    torch.cuda.synchronize()
    us = ev[0].elapsed_time(ev[1]) * 1e3 / steps
    nbytes = sum(w.attend_bytes(t) for t in range(steps)) / steps
    gbs = nbytes / (us * 1e-6) / 1e9
    out["ft_attend"] = {"us_per_layer": round(us, 1), "gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                        "rotary_dim": D, "steps": steps}
    del k_cache, v_cache
    torch.cuda.empty_cache()
    return out


def _best_of(n, fn):
    best = float("inf")
    for _ in range(n):
        t0 = time.perf_counter()
        fn()
        best = min(best, time.perf_counter() - t0)
    return best


def cpu_formats(cores):
    """CPU figures beside ``measure_formats``: the reference's torch ops for
    each legacy format (oracle/cpu_path.py) on host tensors of
    ``format_cases``' shapes cut to 2 layers, GB/s with its byte accounting
    (best of 2 calls; outputs allocated per call, as the reference does)."""
    from oracle import cpu_path

    torch.set_num_threads(cores)
    row, L, bf = 2 * 8 * 128 * 2, 2, torch.bfloat16
    out = {}
    cache = torch.ones((L, 1, 8448, 2, 8, 128), dtype=bf)
    layers = [cache[l, :, :8192] for l in range(L)]
    sec = _best_of(2, lambda: cpu_path.flat_concat(layers))
    out["flat_packet"] = 2 * L * 8192 * row / sec / 1e9
    lens = [int(x) for x in torch.randint(128, 4097, (8,), generator=torch.Generator().manual_seed(0))]
    bcache = torch.ones((L, 8, 4096, 2, 8, 128), dtype=bf)
    dicts = [{l: bcache[l, i:i + 1, :n] for l in range(L)} for i, n in enumerate(lens)]
    sec = _best_of(2, lambda: cpu_path.batch_pad(dicts))
    out["zero_pad_batch"] = L * row * (sum(lens) + 8 * max(lens)) / sec / 1e9
    shards_t = torch.ones((8, L, 8, 4096, 2, 1, 128), dtype=bf)
    shards = [{l: shards_t[j, l] for l in range(L)} for j in range(8)]
    sec = _best_of(2, lambda: cpu_path.concat_dicts(shards))
    out["tp_head_concat"] = 2 * shards_t.numel() * 2 / sec / 1e9
    return {k: {"gbs": round(v, 2), "cores": cores, "kind": "port",
                "sample": "the reference's torch ops on 2 layers of the same shapes"} for k, v in out.items()}


def cpu_ft(cores, w):
    """CPU figures beside ``measure_ft``: the reference's FT prefill write
    (oracle/cpu_path.py ft_store, mha.py:301-306) on 4 of the 64 sequences,
    GB/s; and one FT decode step of the oracle's restatement (the reference
    has no CPU path for it: ft_attention is a CUDA extension) on 2 sequences,
    scaled by attended positions to the whole batch, µs per layer."""
    from oracle import cpu_path, kv_oracle

    torch.set_num_threads(cores)
    B, H, Hq, D, dtype = 4, w.kv_heads, w.q_heads, w.head_dim, w.dtype
    kv = torch.ones((B, 4096, 2, H, D), dtype=dtype)
    k_shape, v_shape = ops.ft_cache_shapes(B, H, 4096, D, dtype)
    k_cache, v_cache = torch.zeros(k_shape, dtype=dtype), torch.zeros(v_shape, dtype=dtype)
    sec = _best_of(2, lambda: cpu_path.ft_store(kv, k_cache, v_cache))
    store_gbs = 2 * kv.numel() * kv.element_size() / sec / 1e9
    nb = 2
    rng = np.random.default_rng(w.seed)
    cap = max(w.lens[:nb]) + 1
    k_ft = rng.standard_normal((nb, H, D // 8, cap, 8)).astype(np.float32)
    v_ft = rng.standard_normal((nb, H, cap, D)).astype(np.float32)
    q = rng.standard_normal((nb, Hq, D)).astype(np.float32)
    new = rng.standard_normal((nb, 2, H, D)).astype(np.float32)
    t0 = time.perf_counter()
    kv_oracle.ft_decode(q, new[:, 0], new[:, 1], k_ft, v_ft, w.lens[:nb], rot_dim=D, dtype="bfloat16")
    sec = time.perf_counter() - t0
    scale = sum(n + 1 for n in w.lens) / sum(n + 1 for n in w.lens[:nb])
    return ({"gbs": round(store_gbs, 2), "cores": cores, "kind": "port",
             "sample": "the reference's FT write (mha.py:301-306) of 4 x 4096 positions"},
            {"us_per_layer": round(sec * scale * 1e6, 1), "cores": 1, "kind": "port",
             "sample": f"the oracle's FT decode step (numpy, fp64) on {nb} sequences, scaled x{scale:.1f} "
                       "(attended positions)"})


def cpu_baseline(w, job, budget_s):
    """The reference's PyTorch ops (oracle/cpu_path.py) on host cores, on a
    bounded sample: 2 layers of pack+unpack and 1 layer x a few decode steps
    of append+attend, at full batch; scaled to the full workload."""
    from oracle import cpu_path

    # Every core this process may run on (the count is reported).
    cores = max(1, len(os.sched_getaffinity(0)))
    torch.set_num_threads(cores)
    n_layers = min(2, w.layers)
    layers = [job.prefill[l].cpu() for l in range(n_layers)]
    # One untimed pass on one layer first, so thread start-up is not timed.
    cpu_path.unpack(cpu_path.pack(layers[:1], w.lens), w.capacity, w.lens)
    t0 = time.perf_counter()
    packed = cpu_path.pack(layers, w.lens)
    t1 = time.perf_counter()
    decode = cpu_path.unpack(packed, w.capacity, w.lens)
    t2 = time.perf_counter()
    pu_bytes = 4 * n_layers * w.live_rows * w.row_bytes
    pu_gbs = pu_bytes / (t2 - t0) / 1e9
    q = job.q[0].cpu()
    kv = job.kv_new[0].cpu()
    steps, step_times = 0, []
    deadline = time.perf_counter() + budget_s
    while steps < min(4, w.decode_steps) and (steps == 0 or time.perf_counter() < deadline):
        s0 = time.perf_counter()
        cpu_path.append(decode[0], kv, [n + steps for n in w.lens])
        cpu_path.attend(q, decode[0], [n + steps + 1 for n in w.lens])
        step_times.append(time.perf_counter() - s0)
        steps += 1
    layer_step = statistics.median(step_times)
    sample = (f"{n_layers} layers pack+unpack ({pu_bytes / 1e9:.2f} GB, after one untimed pass) and {steps} decode steps x 1 layer "
              f"of append+attend, batch {w.batch}; decode_ms_per_step extrapolated x{w.layers} layers")
    # The reference's own setting, one thread (hexgen2/run.py:97): one layer
    # of pack+unpack, and one decode step of one layer over the first
    # sequences of the batch (up to 8), scaled by attended positions.
    torch.set_num_threads(1)
    cpu_path.unpack(cpu_path.pack(layers[:1], w.lens), w.capacity, w.lens)  # untimed warm-up
    s0 = time.perf_counter()
    one = cpu_path.unpack(cpu_path.pack(layers[:1], w.lens), w.capacity, w.lens)
    s1 = time.perf_counter()
    nb = min(8, w.batch)
    sub = [n + 1 for n in w.lens[:nb]]
    s2 = time.perf_counter()
    cpu_path.append(one[0][:nb], kv[:nb], w.lens[:nb])
    cpu_path.attend(q[:nb], one[0][:nb], sub)
    s3 = time.perf_counter()
    scale = sum(n + 1 for n in w.lens) / sum(sub)
    single = {"value": round(2 * w.live_rows * w.row_bytes * 2 / (s1 - s0) / 1e9, 3), "unit": "GB/s", "cores": 1,
              "decode_ms_per_step": round((s3 - s2) * scale * w.layers * 1e3, 1),
              "decode_extrapolated": True,
              "sample": f"1 layer pack+unpack; 1 decode step of 1 layer over {nb} sequences, "
                        f"decode_ms_per_step extrapolated x{scale:.2f} (attended positions) and x{w.layers} layers"}
    torch.set_num_threads(cores)
    return {"value": round(pu_gbs, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": sample, "decode_ms_per_step": round(layer_step * w.layers * 1e3, 1),
            "decode_extrapolated": True, "omp_num_threads_env": os.environ.get("OMP_NUM_THREADS"),
            "pack_s": round(t1 - t0, 3), "unpack_s": round(t2 - t1, 3), "single_thread": single}


SECONDARY = ("tinyllama-1.1b", "llama2-7b", "llama2-70b-tp8")


def measure(w, device, args, steps, warmup, cpu_budget):
    """Build the workload's job, check its full-size handoff, and time
    ``steps`` job passes after ``warmup`` (each pass: pack, unpack, every
    decode step as one graph replay); then the eager decode, the
    MALL-evicted decode (workloads whose handoff fits in the MALL) and the
    CPU baseline.  Returns (result fields, wall seconds of the timed passes)."""
    job = Job(w, device, args.kernel, grid=args.grid, single_launch=not args.two_launch)
    log(f"{w.name}: buffers ready; attention kernel {job.kernel_name}; {job.schedule}")
    if not args.no_verify:
        job.verify()
        log(f"{w.name}: full-size pack/unpack round trip verified")
    n_ev = 4
    job.handoff()
    job.eager_step(0)  # loads every kernel before the graphs are captured
    torch.cuda.synchronize()
    job.capture_graph()
    for _ in range(warmup):
        job.run_graph()
    torch.cuda.synchronize()
    log(f"{w.name}: warmup done")
    # The timed passes are enqueued back to back between two synchronisations
    # (a synchronisation after every pass left the GPU idle before each pack,
    # and the first milliseconds after idling ran 3-7% slow); each pass's
    # events are read afterwards.
    pu_times, pack_times, decode_ms = [], [], []
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(n_ev)] for _ in range(steps)]
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    for k in range(steps):
        job.run_graph(events[k])
        if args.sync_passes:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t_start
    for k, ev in enumerate(events):
        pack_times.append(ev[0].elapsed_time(ev[1]))
        pu_times.append(ev[0].elapsed_time(ev[2]))
        decode_ms.append(ev[2].elapsed_time(ev[3]))
        log(f"{w.name} step {k}: pack+unpack {pu_times[-1]:.3f} ms, decode {decode_ms[-1]:.1f} ms")

    pu_ms = statistics.median(pu_times)
    pu_gbs = w.pack_unpack_bytes() / (pu_ms * 1e-3) / 1e9
    decode_total_ms = sum(decode_ms) / steps
    decode_us_step = decode_total_ms / w.decode_steps * 1e3
    decode_gbs = w.decode_bytes() / (decode_total_ms * 1e-3) / 1e9
    launch_bytes = w.decode_bytes() / (w.layers * w.decode_steps)
    attend_us = decode_total_ms * 1e3 / (w.layers * w.decode_steps)
    achieved = launch_bytes / (attend_us * 1e-6) / 1e9
    # HBM bytes per attention call: not measured in this run (hardware
    # counters need a rocprofv3 --pmc run of their own).  Derived from the
    # committed counter runs (FETCH_SIZE + WRITE_SIZE at decode step 0,
    # calibrated on a plain copy) as their ratio to that step's algorithmic
    # bytes, times this run's average algorithmic bytes per call.
    traffic, traffic_ratio = None, None
    if TRAFFIC_FILE.is_file():
        traffic_ratio = json.loads(TRAFFIC_FILE.read_text()).get(w.name, {}).get("traffic_over_algorithmic")
        if traffic_ratio:
            traffic = int(traffic_ratio * launch_bytes)
    kernels = f"attend_{job.kernel_name}_kernel" + (" + combine_kernel" if job.grid or not job.lists.xcds else "")
    r = {
        "pack_unpack_gbs": round(pu_gbs, 1),
        "pack_unpack_ms": round(pu_ms, 3),
        "pack_unpack_hbm_frac": round(pu_gbs / HBM_PEAK_GBS, 4),
        "pack_ms": round(statistics.median(pack_times), 3),
        "decode_append_attend_us_per_step": round(decode_us_step, 1),
        "decode_gbs": round(decode_gbs, 1),
        "decode_hbm_frac": round(decode_gbs / HBM_PEAK_GBS, 4),
        "roofline": {
            "kernel": f"one hexkv_attend call = {kernels} (fused append+attend, one layer)",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": (f"derived: committed PMC ratio {traffic_ratio} (profiles/traffic.json, decode "
                               "step 0) x this run's algorithmic bytes per call") if traffic else None,
            "bytes_per_launch": int(launch_bytes),
            "avg_launch_us": round(attend_us, 2),
            "timing": "HIP events on the launch stream around the decode phase of every timed pass (all "
                      "its graph replays back to back); avg_launch_us = decode time / (layers x steps), i.e. "
                      "the attention call of one layer with its share of the gaps between launches",
        },
    }
    # Outside the timed passes: the same decode steps launched eagerly, layer
    # by layer, from the host (host gaps included).
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n_ev)]
    job.run(ev)
    torch.cuda.synchronize()
    eager_ms = ev[2].elapsed_time(ev[3])
    r["decode_eager_us_per_step"] = round(eager_ms / w.decode_steps * 1e3, 1)
    log(f"{w.name}: eager decode {eager_ms:.1f} ms")
    if job.mall_flush is not None:
        r["mall"] = ("pack+unpack timed after a 512 MB fill evicts the 256 MB MALL; the decode steps run "
                     "back to back with their working set MALL-resident, decode_mall_evicted_us_per_step "
                     "fills before every step")
        r["decode_mall_evicted_us_per_step"] = round(job.decode_mall_busted(), 1)
    if cpu_budget is not None:
        log(f"{w.name}: cpu baseline")
        r["cpu_baseline"] = cpu_baseline(w, job, cpu_budget)
    r["config"] = {**w.describe(), "attention_kernel": job.kernel_name, "attention_schedule": job.schedule}
    del job
    torch.cuda.empty_cache()
    return r, elapsed


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--workload", default="llama3-8b", choices=WORKLOADS,
                    help="the timed workload (the other GPU workloads follow it unless --no-secondary)")
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU-baseline decode work")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-verify", action="store_true")
    ap.add_argument("--no-formats", action="store_true", help="skip the legacy-format figures")
    ap.add_argument("--no-secondary", action="store_true", help="time only --workload")
    ap.add_argument("--ft", action="store_true", help="add the FasterTransformer-layout figures")
    ap.add_argument("--kernel", default="auto", choices=("auto", "valu", "mfma", "rows"),
                    help="attention kernel (auto: the library's choice for the workload; rows: the "
                         "row-block kernel, work lists only)")
    ap.add_argument("--grid", action="store_true",
                    help="decode attention over the library's uniform partitions instead of work lists")
    ap.add_argument("--two-launch", action="store_true",
                    help="work lists whose split rows a second kernel merges (not planned for the XCDs)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="run only the short dispatch sequence for hardware-counter runs")
    ap.add_argument("--sync-passes", action="store_true",
                    help="synchronise after every timed pass (for kernel traces: rocprofv3 faulted in one of "
                         "its own threads with thousands of graph launches outstanding)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the KV path here runs prefill and decode on one "
              "MI355X; run it with --gpus 1", file=sys.stderr)
        sys.exit(2)
    device = torch.device("cuda", 0)
    w = workload(args.workload)
    log(f"workload {w.describe()}")
    if args.traffic_probe:
        job = Job(w, device, args.kernel, grid=args.grid, single_launch=not args.two_launch)
        log(f"buffers ready; attention kernel {job.kernel_name}; {job.schedule}")
        job.traffic_probe()
        del job
        torch.cuda.empty_cache()
        Job.formats_traffic_probe(device)
        return

    head, elapsed = measure(w, device, args, args.steps, args.warmup,
                            None if args.no_cpu_baseline else args.cpu_budget)
    result = {
        "metric": METRIC,
        "value": head["pack_unpack_gbs"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed * 1e3 / args.steps, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": str(w.dtype).split(".")[-1].replace("bfloat16", "bf16").replace("float16", "fp16"),
        "data": "synthetic (seeded N(0,1) K/V, seeded ragged lengths)",
        "config": {**head.pop("config"), "parallelism": "single GPU (prefill and decode share it)"},
        "cpu_baseline": head.pop("cpu_baseline", None),
    }
    result.update(head)
    if not args.no_secondary:
        # the other GPU configurations, outside the timed job: a few passes each
        steps, warmup = max(1, min(args.steps, 5)), min(args.warmup, 2)
        cpu_budget = None if args.no_cpu_baseline else min(args.cpu_budget, 5.0)
        result["workloads"] = {}
        for name in SECONDARY:
            if name == w.name:
                continue
            r, wall = measure(workload(name), device, args, steps, warmup, cpu_budget)
            r["steps"], r["warmup"], r["ms_per_step"] = steps, warmup, round(wall * 1e3 / steps, 2)
            result["workloads"][name] = r
            log(f"{name}: {r['pack_unpack_gbs']} GB/s pack+unpack, {r['decode_append_attend_us_per_step']} us "
                f"per decode step, attention call {r['roofline']['avg_launch_us']} us ({r['roofline']['frac']})")
    if not args.no_formats:
        result["formats"] = measure_formats(device)
        log(f"legacy formats {result['formats']}")
        if args.ft:
            result["ft_layout"] = measure_ft(device)
            log(f"FT layout {result['ft_layout']}")
        if not args.no_cpu_baseline:
            cores = result["cpu_baseline"]["cores"]
            for name, cpu in cpu_formats(cores).items():
                result["formats"][name]["cpu"] = cpu
            if args.ft:
                store_cpu, attend_cpu = cpu_ft(cores, workload("llama3-8b"))
                result["ft_layout"]["ft_store"]["cpu"] = store_cpu
                result["ft_layout"]["ft_attend"]["cpu"] = attend_cpu
            log("CPU formats done")
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
