"""The two-rank prefill/decode pilot (hexgen2_amd.run) with both ranks on one
GPU, launched as the reference's runtime test launches its pilot
(tests/test_runtime.py:21-39 of the reference): the reference's trace
(configs/tiny-trace.jsonl) on the seed-17 fixture with one warmup request.

Checks the reference's assertions -- output token counts [1, 1, 4, 3] with
warmup first, every colocated check matching, positive packet bytes, a final
"complete" event per rank, and a retry refusing to overwrite the records --
plus this build's: the exact packet bytes, the KV handoff through device
memory, and greedy tokens equal to HuggingFace full-context recompute
(tests/golden/trace_tokens.json) in float16 and float32."""
import json
import os
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
TOKENS = json.loads((GOLDEN / "trace_tokens.json").read_text())


def launch(output, *extra, timeout=240):
    env = dict(os.environ, HSA_ENABLE_IPC_MODE_LEGACY="0", PYTHONPATH=str(ROOT))
    cmd = [sys.executable, "-m", "torch.distributed.run", "--standalone", "--local-addr", "127.0.0.1",
           "--nproc_per_node=2", "-m", "hexgen2_amd.run", "--model-dir", str(GOLDEN / "fixture_seed17"),
           "--trace", str(GOLDEN / "tiny-trace.jsonl"), "--output", str(output), "--check-colocated", *extra]
    print("launch:", " ".join(cmd[3:]), flush=True)
    return subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=timeout)


def check_records(output, dtype_bytes, golden):
    records = [json.loads(s) for s in (output / "requests.jsonl").read_text().splitlines()]
    assert [r["output_tokens"] for r in records] == [1, 1, 4, 3]
    assert [r["warmup"] for r in records] == [True, False, False, False]
    assert all(r["colocated_matches"] for r in records)
    for r in records:
        # int64 first token + 2 layers x L x (2 x 2 KV heads x 32 dims)
        assert r["kv_packet_bytes"] == 8 + 2 * r["input_tokens"] * 2 * 2 * 32 * dtype_bytes
        if golden and not r["warmup"]:
            assert r["token_ids"] == TOKENS[r["id"]]["hf_fp32_tokens"], r["id"]
    for rank in (0, 1):
        events = [json.loads(s) for s in (output / f"rank-{rank}-events.jsonl").read_text().splitlines()]
        assert events[-1]["event"] == "complete", events[-1]
    return records


@pytest.mark.timeout(600)
def test_pilot_device_memory_handoff_float16(tmp_path):
    result = launch(tmp_path / "out")
    assert result.returncode == 0, result.stderr[-4000:]
    records = check_records(tmp_path / "out", 2, golden=True)
    assert all(r["handoff"] == "device memory (IPC)" for r in records)
    retry = launch(tmp_path / "out", timeout=120)
    assert retry.returncode != 0
    assert "Refusing to overwrite" in retry.stderr


@pytest.mark.timeout(600)
def test_pilot_bfloat16_fused_append(tmp_path):
    result = launch(tmp_path / "out", "--dtype", "bfloat16", "--fused-append")
    assert result.returncode == 0, result.stderr[-4000:]
    check_records(tmp_path / "out", 2, golden=False)


@pytest.mark.timeout(600)
def test_pilot_float32_host_wire(tmp_path):
    result = launch(tmp_path / "out", "--dtype", "float32", "--wire", "--profile-first")
    assert result.returncode == 0, result.stderr[-4000:]
    records = check_records(tmp_path / "out", 4, golden=True)
    assert all(r["handoff"] == "host wire" for r in records)
    for rank in (0, 1):
        assert (tmp_path / "out" / f"rank-{rank}-trace.json.gz").is_file()
