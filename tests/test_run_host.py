"""Host logic of the pilot runner (no GPU): trace validation, the warmup
schedule and the refusal to overwrite an earlier run's records."""
import json
from pathlib import Path
from types import SimpleNamespace

import pytest

from hexgen2_amd.run import Pilot, RankLog, Request, read_trace


GOLDEN = Path(__file__).resolve().parent / "golden"


def write(tmp_path, rows):
    path = tmp_path / "trace.jsonl"
    path.write_text("\n".join(json.dumps(r) for r in rows) + "\n")
    return path


def test_reference_trace_reads_in_order():
    reqs = read_trace(GOLDEN / "tiny-trace.jsonl", GOLDEN / "fixture_seed17", 128, 128)
    assert [(r.id, len(r.input_ids), r.max_new_tokens, r.warmup) for r in reqs] == [
        ("one-token", 1, 1, False), ("short", 4, 4, False), ("longer", 7, 3, False)]


@pytest.mark.parametrize("rows,match", [
    ([], "empty"),
    ([{"id": "a", "input_ids": [1], "max_new_tokens": 1}, {"id": "a", "input_ids": [2], "max_new_tokens": 1}],
     "unique"),
    ([{"id": "__warmup_0", "input_ids": [1], "max_new_tokens": 1}], "unique"),
    ([{"id": "a", "input_ids": [1], "max_new_tokens": 1, "arrival": 0.5}], "unsupported"),
    ([{"id": "a", "input_ids": [1], "prompt": "x", "max_new_tokens": 1}], "exactly one"),
    ([{"id": "a", "input_ids": [1], "max_new_tokens": 1, "warmup": 1}], "boolean"),
    ([{"id": "a", "input_ids": [], "max_new_tokens": 1}], "nonempty"),
    ([{"id": "a", "input_ids": [500], "max_new_tokens": 1}], "below 128"),
    ([{"id": "a", "input_ids": [1], "max_new_tokens": 0}], "max_new_tokens"),
    ([{"id": "a", "input_ids": [1] * 120, "max_new_tokens": 9}], "context"),
])
def test_invalid_traces_are_rejected(tmp_path, rows, match):
    with pytest.raises(ValueError, match=match):
        read_trace(write(tmp_path, rows), GOLDEN / "fixture_seed17", 128, 128)


def test_warmup_schedule_repeats_the_first_request():
    pilot = Pilot.__new__(Pilot)
    pilot.args = SimpleNamespace(warmup=2)
    pilot.requests = [Request("x", [1, 2], 3), Request("y", [4], 1)]
    sched = pilot.schedule()
    assert [(r.id, r.warmup) for r in sched] == [("__warmup_0", True), ("__warmup_1", True),
                                                 ("x", False), ("y", False)]
    assert sched[0].input_ids == [1, 2] and sched[0].max_new_tokens == 3


def test_rank_log_refuses_to_overwrite(tmp_path):
    log = RankLog(tmp_path, 0)
    log.event("start")
    log.event("complete")
    events = [json.loads(s) for s in (tmp_path / "rank-0-events.jsonl").read_text().splitlines()]
    assert [e["event"] for e in events] == ["start", "complete"]
    assert all("utc_ns" in e and "monotonic_ns" in e for e in events)
    with pytest.raises(FileExistsError, match="Refusing to overwrite"):
        RankLog(tmp_path, 0)
    RankLog(tmp_path, 1)  # the other rank's log is separate
