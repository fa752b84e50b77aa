"""Two-rank prefill/decode pilot on one GPU, with the KV handoff in device memory.

Rank 0 owns prefill, rank 1 owns decode; both processes drive the same GPU.
For every request of a JSONL trace, rank 0 prefills, packs the live KV rows
(one hexkv launch) and sends them with the first token; rank 1 unpacks them
into its decode cache, decodes greedily and replies with the tokens.  The
KV bytes never leave HBM: rank 1 maps rank 0's packed buffer through a HIP
IPC handle (``IpcChannel``); only the packet header and the handles cross
the host (Gloo).  ``--wire`` sends the payload through host memory instead,
as the reference's transport does.

Behaviour kept from the reference pilot runner (hexgen2/run.py), because
its runtime test asserts it (tests/test_runtime.py:28-39 of the reference):
the command line, a ``requests.jsonl`` record per request with
``output_tokens``, ``warmup``, ``colocated_matches`` and ``kv_packet_bytes``,
per-rank ``rank-<r>-events.jsonl`` ending in a ``complete`` event, a
``rank-<r>-trace.json.gz`` with ``--profile-first``, and a refusal to
overwrite the records of an earlier run.  Launch with two processes:

    python -m torch.distributed.run --standalone --local-addr 127.0.0.1 \\
        --nproc_per_node 2 -m hexgen2_amd.run --model-dir M --trace T --output O
"""
from __future__ import annotations

import argparse
import contextlib
import gzip
import hashlib
import json
import os
import shutil
import time
import traceback
from dataclasses import asdict, dataclass
from datetime import timedelta
from pathlib import Path
from typing import List, Optional

import torch
import torch.distributed as dist

from .engine import Engine
from .transport import IpcChannel, recv_packet, send_packet

PREFILL_RANK, DECODE_RANK = 0, 1
TRACE_FIELDS = {"id", "prompt", "input_ids", "max_new_tokens", "warmup"}


def now() -> dict:
    """Wall-clock and monotonic nanoseconds, for records and latencies."""
    return {"utc_ns": time.time_ns(), "monotonic_ns": time.monotonic_ns()}


def elapsed_ms(start: dict, end: dict) -> float:
    return (end["monotonic_ns"] - start["monotonic_ns"]) / 1e6


@dataclass
class Request:
    id: str
    input_ids: List[int]
    max_new_tokens: int
    warmup: bool = False

    def metadata(self) -> dict:
        """What the prefill rank sends with the KV packet."""
        return {"id": self.id, "prompt_length": len(self.input_ids)}


def read_trace(path: Path, model_dir: Path, context_limit: int, vocab_size: int) -> List[Request]:
    """The trace's requests, in order.  A request names a unique id, its prompt
    as ``input_ids`` or as ``prompt`` text (tokenised with the model's own
    tokenizer), ``max_new_tokens`` >= 1 within the context limit, and an
    optional boolean ``warmup``; anything else is rejected before any GPU
    work starts."""
    requests: List[Request] = []
    tokenizer = None
    for number, line in enumerate(Path(path).read_text().splitlines(), start=1):
        if not line.strip():
            continue
        row = json.loads(line)
        where = f"{path}:{number}"
        rid = row.get("id")
        if not isinstance(rid, str) or not rid or rid.startswith("__warmup_"):
            raise ValueError(f"{where}: every request must have a unique string id")
        if any(r.id == rid for r in requests):
            raise ValueError(f"{where}: every request must have a unique string id ({rid!r} repeats)")
        extra = set(row) - TRACE_FIELDS
        if extra:
            raise ValueError(f"{where}: unsupported workload fields {sorted(extra)}; the pilot does not "
                             "schedule arrivals or sampling")
        if ("prompt" in row) == ("input_ids" in row):
            raise ValueError(f"{where}: specify exactly one of prompt/input_ids")
        warmup = row.get("warmup", False)
        if not isinstance(warmup, bool):
            raise ValueError(f"{where}: warmup must be a boolean")
        ids = row.get("input_ids")
        if ids is None:
            if not isinstance(row["prompt"], str):
                raise ValueError(f"{where}: prompt must be text")
            if tokenizer is None:
                from transformers import AutoTokenizer
                tokenizer = AutoTokenizer.from_pretrained(model_dir, local_files_only=True)
            ids = tokenizer.encode(row["prompt"], add_special_tokens=True)
        if not isinstance(ids, list) or not ids or not all(type(i) is int and 0 <= i < vocab_size for i in ids):
            raise ValueError(f"{where}: input_ids must be a nonempty list of token ids below {vocab_size}")
        count = row.get("max_new_tokens")
        if type(count) is not int or count < 1 or len(ids) + count > context_limit:
            raise ValueError(f"{where}: max_new_tokens must be >= 1 and fit the {context_limit}-token context")
        requests.append(Request(rid, list(ids), count, warmup))
    if not requests:
        raise ValueError(f"{path}: the workload is empty")
    return requests


class RankLog:
    """Append-only JSONL event log of one rank, written through to disk."""

    def __init__(self, folder: Path, rank: int):
        self.path = folder / f"rank-{rank}-events.jsonl"
        self.rank = rank
        if self.path.exists():
            raise FileExistsError(f"Refusing to overwrite rank records in {folder}; use a fresh run directory")

    @staticmethod
    def write(path: Path, record: dict) -> None:
        with path.open("a") as f:
            f.write(json.dumps(record, allow_nan=False) + "\n")
            f.flush()
            os.fsync(f.fileno())

    def event(self, name: str, **fields) -> None:
        self.write(self.path, {"event": name, "rank": self.rank, **fields, **now()})


class Profiled(contextlib.AbstractContextManager):
    """torch.profiler around one request, exported as rank-<r>-trace.json.gz."""

    def __init__(self, target: Optional[Path]):
        self.target = target
        self.profiler = None

    def __enter__(self):
        if self.target is not None:
            acts = [torch.profiler.ProfilerActivity.CPU, torch.profiler.ProfilerActivity.CUDA]
            self.profiler = torch.profiler.profile(activities=acts, record_shapes=True, profile_memory=True)
            self.profiler.start()
        return self

    def __exit__(self, *exc):
        if self.profiler is not None:
            self.profiler.stop()
            raw = self.target.with_suffix("")  # rank-<r>-trace.json
            self.profiler.export_chrome_trace(str(raw))
            with raw.open("rb") as src, gzip.open(self.target, "wb") as dst:
                shutil.copyfileobj(src, dst)
            raw.unlink()
        return False


class Pilot:
    """One rank of the pilot: the request loop and the role-specific halves."""

    def __init__(self, args, rank: int, log: RankLog):
        self.args, self.rank, self.log = args, rank, log
        self.handoff = "host wire" if args.wire else "device memory (IPC)"
        self.channel = None if args.wire else IpcChannel()
        self.engine = Engine(args.model_dir, args.engine, "cuda", args.dtype, fused_append=args.fused_append)
        cfg = self.engine.config
        self.requests = read_trace(args.trace, args.model_dir, cfg.max_position_embeddings, cfg.vocab_size)

    def settings_digest(self) -> str:
        """What both ranks must agree on before the first request."""
        trace = json.dumps([asdict(r) for r in self.requests], sort_keys=True)
        settings = {k: getattr(self.args, k) for k in ("engine", "dtype", "seed", "warmup", "profile_first",
                                                        "fused_append", "wire")}
        settings["trace_sha256"] = hashlib.sha256(trace.encode()).hexdigest()
        settings["model"] = self.engine.identity["sha256"]
        return hashlib.sha256(json.dumps(settings, sort_keys=True).encode()).hexdigest()

    def schedule(self) -> List[Request]:
        """Warmup copies of the first request, then the trace."""
        first = self.requests[0]
        warm = [Request(f"__warmup_{i}", first.input_ids, first.max_new_tokens, True)
                for i in range(self.args.warmup)]
        return warm + self.requests

    # -- prefill rank ---------------------------------------------------------
    def prefill_side(self, index: int, req: Request, profiled: bool) -> None:
        t0 = now()
        first, cache, _ = self.engine.prefill(req.input_ids, req.max_new_tokens)
        self.engine.synchronize()
        t1 = now()
        tensors = {"first": first, **{str(layer): kv for layer, kv in cache.items()}}
        nbytes = send_packet(tensors, req.metadata(), dst=DECODE_RANK, channel=self.channel)
        self.engine.synchronize()
        t2 = now()
        answer, reply = recv_packet(src=DECODE_RANK, channel=self.channel)
        t3 = now()
        tokens = answer["tokens"].cpu().tolist()
        del answer, tensors, cache, first
        if reply.get("id") != req.id or len(tokens) != req.max_new_tokens:
            raise ValueError(f"request {req.id}: the decode rank answered {reply.get('id')!r} with "
                             f"{len(tokens)} tokens, expected {req.max_new_tokens}")
        record = {"id": req.id, "index": index, "warmup": req.warmup, "profiled": profiled,
                  "engine": self.args.engine, "handoff": self.handoff, "input_tokens": len(req.input_ids),
                  "output_tokens": len(tokens), "token_ids": tokens, "kv_packet_bytes": nbytes,
                  "start": t0, "prefill_end": t1, "send_end": t2, "end": t3,
                  "prefill_ms": elapsed_ms(t0, t1), "send_ms": elapsed_ms(t1, t2),
                  "roundtrip_ms": elapsed_ms(t0, t3), "decode": reply, "status": "success",
                  "timing_note": "requests run one after another; latencies are per request, not serving throughput"}
        if self.args.check_colocated:
            # The same engine without a handoff must produce the same tokens.
            f, c, _ = self.engine.prefill(req.input_ids, req.max_new_tokens)
            local = self.engine.decode(f, c, len(req.input_ids), req.max_new_tokens)
            record["colocated_token_ids"] = local
            record["colocated_matches"] = local == tokens
            if local != tokens:
                record["status"] = "correctness_failure"
        RankLog.write(self.args.output / "requests.jsonl", record)
        if record["status"] != "success":
            raise ValueError(f"request {req.id}: transferred-cache output differs from colocated inference")

    # -- decode rank ----------------------------------------------------------
    def decode_side(self, index: int, req: Request, profiled: bool) -> None:
        tensors, meta = recv_packet(src=PREFILL_RANK, channel=self.channel)
        self.engine.synchronize()
        t0 = now()
        if meta != req.metadata():
            raise ValueError(f"request {req.id}: prefill metadata {meta} does not match the trace")
        marks = []

        def on_token(token):
            self.engine.synchronize()
            marks.append({"token_id": token, **now()})

        first = tensors.pop("first")
        layers = {int(name): kv for name, kv in tensors.items()}
        tokens = self.engine.decode(first, layers, len(req.input_ids), req.max_new_tokens, on_token)
        t1 = now()
        # The received views alias the prefill rank's memory: release (unmap)
        # them before answering, so it may free its packet.
        del tensors, layers, first
        reply = {"id": req.id, "receive_end": t0, "decode_end": t1, "token_events": marks,
                 "decode_ms": elapsed_ms(t0, t1)}
        self.log.event("decode_complete", **reply)
        send_packet({"tokens": torch.tensor(tokens, dtype=torch.long, device="cuda")}, reply,
                    dst=PREFILL_RANK, channel=self.channel)

    def run(self) -> None:
        digests = [None, None]
        dist.all_gather_object(digests, self.settings_digest())
        if digests[0] != digests[1]:
            raise ValueError("the prefill and decode ranks were started with different traces, models or settings")
        (self.args.output / f"rank-{self.rank}-workload.json").write_text(
            json.dumps([asdict(r) for r in self.requests], indent=2) + "\n")
        self.log.event("ready", handoff=self.handoff, model_identity=self.engine.identity,
                       gpu={"name": torch.cuda.get_device_name(), "index": self.args.gpu,
                            "allocated_bytes": torch.cuda.memory_allocated()})
        serve = self.prefill_side if self.rank == PREFILL_RANK else self.decode_side
        profile_pending = self.args.profile_first
        for index, req in enumerate(self.schedule()):
            dist.barrier()
            self.engine.synchronize()
            profiled = profile_pending and not req.warmup
            profile_pending = profile_pending and not profiled
            target = self.args.output / f"rank-{self.rank}-trace.json.gz" if profiled else None
            self.log.event("request_start", id=req.id, index=index)
            with Profiled(target), torch.profiler.record_function(f"hexgen2_amd.{serve.__name__}"):
                serve(index, req, profiled)
            self.log.event("request_complete", id=req.id,
                           peak_gpu_allocated_bytes=torch.cuda.max_memory_allocated())
        dist.barrier()


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--model-dir", type=Path, required=True)
    ap.add_argument("--trace", type=Path, required=True)
    ap.add_argument("--output", type=Path, default=os.environ.get("HEXGEN2_RUN_DIR"))
    ap.add_argument("--engine", choices=["native"], default="native")
    ap.add_argument("--dtype", choices=["float16", "bfloat16", "float32"], default="float16")
    ap.add_argument("--gpu", type=int, default=0, help="the one GPU both ranks use")
    ap.add_argument("--seed", type=int, default=123)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--timeout", type=int, default=180)
    ap.add_argument("--fused-append", action="store_true", help="decode with the fused append+attend launch")
    ap.add_argument("--wire", action="store_true",
                    help="send KV payloads through host memory over the process group (reference path)")
    ap.add_argument("--check-colocated", action="store_true",
                    help="compare every output to the same engine without a KV transfer")
    ap.add_argument("--profile-first", action="store_true",
                    help="export a profiler trace of the first measured request")
    args = ap.parse_args(argv)
    if args.output is None:
        ap.error("--output (or HEXGEN2_RUN_DIR) is required")
    return args


def main(argv=None) -> None:
    args = parse_args(argv)
    args.output.mkdir(parents=True, exist_ok=True)
    rank = int(os.environ.get("RANK", "-1"))
    log = RankLog(args.output, rank)
    log.event("start", pid=os.getpid(), run_id=os.environ.get("HEXGEN2_RUN_ID"),
              arguments={k: str(v) if isinstance(v, Path) else v for k, v in vars(args).items()})
    try:
        if int(os.environ.get("WORLD_SIZE", "0")) != 2:
            raise ValueError("The pilot runs exactly two ranks (prefill and decode)")
        if args.warmup < 0:
            raise ValueError("--warmup must be nonnegative")
        torch.cuda.set_device(args.gpu)
        torch.set_num_threads(1)
        torch.manual_seed(args.seed)
        torch.backends.cuda.matmul.allow_tf32 = False
        # Control messages, packet headers and (with --wire) payloads: Gloo.
        dist.init_process_group("gloo", timeout=timedelta(seconds=args.timeout))
        Pilot(args, rank, log).run()
        log.event("complete")
    except BaseException as error:
        log.event("failure", error_type=type(error).__name__, message=str(error),
                  traceback=traceback.format_exc())
        raise
    finally:
        if dist.is_initialized():
            dist.destroy_process_group()


if __name__ == "__main__":
    main()
