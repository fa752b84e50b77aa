"""Two-process KV handoff on one GPU, at a workload's full size.

The two-rank pilot (hexgen2/run.py:141-198) hands each request's KV packet
from the prefill rank to the decode rank; the reference moves it through
host memory and TCP (hexgen2/transport.py:44-100).  Here rank 0 packs the
prefill cache into one packet tensor per layer and sends it through
``IpcChannel``: the header goes over a Gloo group, the bytes stay where rank
0's pack kernel wrote them.  As in ``Engine.prefill``, a packet below 1 GiB
is one packed allocation whose layers are views (one handle export, one
mapping), a larger one one allocation per layer (each below the 2 GiB IPC
limit).
Rank 1 maps them and unpacks straight from rank 0's memory into its decode
cache.  Per round, one JSON line per rank:

* rank 0: ``send_ms``, the sender's time in ``send_packet``;
* rank 1: ``handoff_ms`` (rank 0's send start to the tensors being usable on
  rank 1, both on the host's monotonic clock), the unpack time and rate
  (bytes read + written) from the peer's memory and from a local copy of the
  same packet, and whether a sampled sequence arrived bit-exact.

    python -m hexgen2_amd.handoff_bench [--workload llama3-8b] [--rounds 3]

Synthetic data (seeded N(0, 1)); the decode rank holds the decode cache and,
for the local comparison, a copy of the packet (Llama-3-8B: 68 + 32 GB on
rank 1, 32 GB on rank 0 after its prefill cache is freed).
"""
from __future__ import annotations

import argparse
import json
import os
import tempfile
import time
from datetime import timedelta
from pathlib import Path

import torch
import torch.distributed as dist
import torch.multiprocessing as mp


def _worker(rank: int, rendezvous: str, workload_name: str, rounds: int) -> None:
    from . import ops
    from .engine import PER_LAYER_HANDOFF_BYTES
    from .transport import IpcChannel, recv_packet, send_packet
    from .workloads import workload

    torch.cuda.set_device(0)
    dist.init_process_group("gloo", rank=rank, world_size=2, init_method=Path(rendezvous).as_uri(),
                            timeout=timedelta(seconds=120))
    channel = IpcChannel()
    w = workload(workload_name)
    L, shape = w.layers, (w.batch, w.capacity, 2, w.kv_heads, w.head_dim)
    rows, cu = w.live_rows, [0]
    for n in w.lens:
        cu.append(cu[-1] + n)
    nbytes = 2 * L * rows * w.row_bytes
    try:
        if rank == 0:
            g = torch.Generator(device="cuda").manual_seed(w.seed + 1)
            prefill = [torch.empty(shape, dtype=w.dtype, device="cuda").normal_(generator=g) for _ in range(L)]
            if L * rows * w.row_bytes < PER_LAYER_HANDOFF_BYTES:
                packed = list(torch.empty((L, rows, *shape[2:]), dtype=w.dtype, device="cuda").unbind(0))
            else:
                packed = [torch.empty((rows, *shape[2:]), dtype=w.dtype, device="cuda") for _ in range(L)]
            ops.pack_live(prefill, w.lens, out=packed)
            torch.cuda.synchronize()
            del prefill
            torch.cuda.empty_cache()
            for rnd in range(rounds):
                dist.barrier()
                t0 = time.monotonic_ns()
                send_packet({str(l): packed[l] for l in range(L)}, {"t0": t0, "round": rnd}, dst=1, channel=channel)
                t1 = time.monotonic_ns()
                reply, _ = recv_packet(src=1, channel=channel)  # rank 1 is done with the packet
                del reply
                print(json.dumps({"rank": 0, "workload": w.name, "round": rnd, "send_ms": round((t1 - t0) / 1e6, 3),
                                  "layers": L, "packet_bytes": L * rows * w.row_bytes,
                                  "allocations": len({t.untyped_storage().data_ptr() for t in packed})}), flush=True)
        else:
            decode = [torch.empty(shape, dtype=w.dtype, device="cuda") for _ in range(L)]
            local = None
            for rnd in range(rounds):
                dist.barrier()
                tensors, meta = recv_packet(src=0, channel=channel)
                received = time.monotonic_ns()
                mapped = [tensors[str(l)] for l in range(L)]
                ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
                ev[0].record()
                ops.unpack_live(mapped, decode, w.lens)
                ev[1].record()
                torch.cuda.synchronize()
                if local is None:
                    local = [m.clone() for m in mapped]
                ev[2].record()
                ops.unpack_live(local, decode, w.lens)
                ev[3].record()
                torch.cuda.synchronize()
                b, l = len(w.lens) // 2, L // 2
                exact = torch.equal(decode[l][b, :w.lens[b]].view(torch.uint8),
                                    mapped[l][cu[b]:cu[b + 1]].view(torch.uint8))
                peer_ms, local_ms = ev[0].elapsed_time(ev[1]), ev[2].elapsed_time(ev[3])
                print(json.dumps({"rank": 1, "workload": w.name, "round": rnd,
                                  "handoff_ms": round((received - meta["t0"]) / 1e6, 3),
                                  "unpack_from_peer_ms": round(peer_ms, 3),
                                  "unpack_from_peer_gbs": round(nbytes / peer_ms / 1e6, 1),
                                  "unpack_local_ms": round(local_ms, 3),
                                  "unpack_local_gbs": round(nbytes / local_ms / 1e6, 1),
                                  "sampled_sequence_bit_exact": bool(exact)}), flush=True)
                del tensors, mapped
                send_packet({"done": torch.zeros(1, device="cuda")}, {"round": rnd}, dst=0, channel=channel)
        dist.barrier()
    finally:
        dist.destroy_process_group()


def main() -> None:
    from .workloads import WORKLOADS

    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--workload", default="llama3-8b", choices=WORKLOADS)
    ap.add_argument("--rounds", type=int, default=3)
    args = ap.parse_args()
    os.environ.setdefault("HSA_ENABLE_IPC_MODE_LEGACY", "0")
    with tempfile.TemporaryDirectory() as tmp:
        mp.spawn(_worker, args=(str(Path(tmp) / "rendezvous"), args.workload, args.rounds), nprocs=2, join=True)


if __name__ == "__main__":
    main()
