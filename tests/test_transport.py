"""Handoff transport: the reference's own transport vectors (tests/test_transport.py
of the reference: lossless two-process round trip of a non-contiguous and a
constant KV layer in fp16/bf16/fp32 with layer order [7, 2], token [42, 17];
header rejection of shapes [-1], [True], [2**40], [1]*9 and of duplicate
names), run against this package's wire protocol over Gloo on the CPU, plus
the byte-exact packet header the reference's send_packet puts on the wire
(hexgen2/transport.py:45-55) for that fixture."""
import json
from datetime import timedelta
from pathlib import Path

import pytest
import torch
import torch.distributed as dist
import torch.multiprocessing as mp

from hexgen2_amd.transport import (DeviceChannel, _encode_header, recv_data, recv_packet, send_data,
                                   send_packet, validate_header)

GOLDEN = Path(__file__).resolve().parent / "golden"


def fixture_cache(dtype):
    return {7: torch.arange(-24, 24).reshape(1, 4, 2, 2, 3).to(dtype)[..., ::2],
            2: torch.full((1, 3, 2, 1, 4), -1.25, dtype=dtype)}


def _echo_peer(rank, rendezvous, failures):
    """Two processes over Gloo: rank 0 sends each dtype's fixture
    (send_data), rank 1 receives it and sends back exactly what it got, rank
    0 receives the echo.  Both sides check what they received against the
    fixture bit for bit; then one send_packet/recv_packet with an empty
    tensor and metadata.  Failures go to the parent through ``failures``."""
    torch.set_num_threads(1)
    dist.init_process_group("gloo", rank=rank, world_size=2, init_method=Path(rendezvous).as_uri(),
                            timeout=timedelta(seconds=30))
    peer = 1 - rank
    token = torch.tensor([42, 17], dtype=torch.long)
    try:
        for dtype in (torch.float16, torch.bfloat16, torch.float32):
            cache = fixture_cache(dtype)
            if rank == 1:  # echo side: receive, then return what arrived
                got_token, got_cache = recv_data(src=peer, num_layers=len(cache))
                send_data(got_token, got_cache, dst=peer)
            else:
                send_data(token, cache, dst=peer)
                got_token, got_cache = recv_data(src=peer, num_layers=len(cache))
            assert list(got_cache) == [7, 2], f"{dtype}: layer order {list(got_cache)}"
            assert torch.equal(got_token, token), f"{dtype}: token {got_token}"
            for layer, want in cache.items():
                assert got_cache[layer].dtype == want.dtype and torch.equal(got_cache[layer], want), \
                    f"{dtype}: layer {layer} changed on the wire"
        if rank == 0:
            send_packet({"a": torch.zeros((0, 3)), "b": torch.tensor([1.5])}, {"id": "r1"}, dst=peer)
        else:
            tensors, meta = recv_packet(src=peer)
            assert meta == {"id": "r1"} and tuple(tensors["a"].shape) == (0, 3)
            assert torch.equal(tensors["b"], torch.tensor([1.5]))
    except Exception as error:  # reported by the parent with the rank that saw it
        failures.put((rank, repr(error)))
        raise
    finally:
        dist.destroy_process_group()


def test_lossless_real_process_roundtrip(tmp_path):
    ctx = mp.get_context("spawn")
    failures = ctx.SimpleQueue()
    procs = [ctx.Process(target=_echo_peer, args=(r, str(tmp_path / "rendezvous"), failures)) for r in (0, 1)]
    for p in procs:
        p.start()
    for p in procs:
        p.join(120)
    seen = []
    while not failures.empty():
        seen.append(failures.get())
    assert not seen, seen
    assert [p.exitcode for p in procs] == [0, 0]


@pytest.mark.parametrize("shape", [[-1], [True], [2 ** 40], [1] * 9])
def test_invalid_shapes_are_rejected_before_allocating_payload(shape):
    with pytest.raises(ValueError):
        validate_header({"version": 1, "tensors": [{"name": "x", "shape": shape, "dtype": "torch.float32"}]})


def test_duplicate_names_and_bad_headers_are_rejected():
    with pytest.raises(ValueError):
        validate_header({"version": 1, "tensors": [
            {"name": "x", "shape": [1], "dtype": "torch.float32"},
            {"name": "x", "shape": [1], "dtype": "torch.float32"}]})
    with pytest.raises(ValueError):
        validate_header({"version": 2, "tensors": []})
    with pytest.raises(ValueError):
        validate_header({"version": 1, "tensors": [{"name": "x", "shape": [1], "dtype": "torch.complex64"}]})
    with pytest.raises(ValueError):
        validate_header({"version": 1, "tensors": [{"name": 3, "shape": [1], "dtype": "torch.float32"}]})
    too_many = [{"name": str(i), "shape": [1], "dtype": "torch.uint8"} for i in range(1025)]
    with pytest.raises(ValueError):
        validate_header({"version": 1, "tensors": too_many})
    # the 8 GiB wire limit (transport.py:18, 39-40): exactly 8 GiB passes, one byte more fails
    assert validate_header({"version": 1, "tensors": [{"name": "x", "shape": [8, 1024 ** 3],
                                                       "dtype": "torch.uint8"}]}) == 8 * 1024 ** 3
    with pytest.raises(ValueError):
        validate_header({"version": 1, "tensors": [{"name": "x", "shape": [8 * 1024 ** 3 + 1],
                                                    "dtype": "torch.uint8"}]})


def test_payload_accounting_matches_reference_evidence():
    # kv_packet_bytes the reference recorded for its fixture: int64 token +
    # 2 layers x [1, L, 2, 2, 32] fp16 (evidence/2026-10-19/fabric-pilot.json:81, 98, 114)
    cases = json.loads((GOLDEN / "packet_bytes.json").read_text())["cases"]
    for c in cases:
        header = {"version": 1, "metadata": {}, "tensors": [{"name": "first", "shape": [1], "dtype": "torch.int64"}] + [
            {"name": str(l), "shape": [1, c["prompt_tokens"], 2, c["kv_heads"], c["head_dim"]],
             "dtype": "torch.float16"} for l in range(c["layers"])]}
        assert validate_header(header) == c["kv_packet_bytes"]


def test_header_bytes_match_the_reference_wire_format():
    cache = fixture_cache(torch.float16)
    tensors = {"token": torch.tensor([42, 17]), **{f"kv/{k}": v for k, v in cache.items()}}
    encoded, payload = _encode_header(tensors, {"layers": [7, 2]}, 8 * 1024 ** 3)
    want = (b'{"version": 1, "metadata": {"layers": [7, 2]}, "tensors": ['
            b'{"name": "token", "shape": [2], "dtype": "torch.int64"}, '
            b'{"name": "kv/7", "shape": [1, 4, 2, 2, 2], "dtype": "torch.float16"}, '
            b'{"name": "kv/2", "shape": [1, 3, 2, 1, 4], "dtype": "torch.float16"}]}')
    assert encoded == want
    assert payload == 2 * 8 + 32 * 2 + 24 * 2


def test_device_channel_keeps_wire_validation_on_cpu_tensors():
    # the same-GPU carrier parses and checks the header exactly as the wire does
    a, b = DeviceChannel.pair()
    cache = fixture_cache(torch.bfloat16)
    assert send_data(torch.tensor([42, 17]), cache, dst=1, channel=a) == 2 * 8 + 32 * 2 + 24 * 2
    token, returned = recv_data(src=0, num_layers=2, channel=b)
    assert list(returned) == [7, 2] and token.tolist() == [42, 17]
    for key in cache:
        torch.testing.assert_close(returned[key], cache[key], rtol=0, atol=0)
    with pytest.raises(ValueError):
        send_data(torch.tensor([1]), {"7": cache[7]}, dst=1, channel=a)  # non-int layer key
    send_data(torch.tensor([1]), cache, dst=1, channel=a)
    with pytest.raises(ValueError):
        recv_data(src=0, num_layers=3, channel=b)
    with pytest.raises(RuntimeError):
        recv_packet(src=0, channel=b)  # nothing queued
    limited, peer = DeviceChannel.pair(max_payload=100)
    with pytest.raises(ValueError):
        send_packet({"x": torch.zeros(101, dtype=torch.uint8)}, {}, dst=1, channel=limited)


def _ipc_control_peer(rank, rendezvous, failures):
    """Rank 0 hand-crafts IpcChannel control messages; rank 1's recv must
    reject each before it maps anything (no GPU is touched)."""
    from hexgen2_amd.transport import IpcChannel
    torch.set_num_threads(1)
    dist.init_process_group("gloo", rank=rank, world_size=2, init_method=Path(rendezvous).as_uri(),
                            timeout=timedelta(seconds=30))
    header, _ = _encode_header({"x": torch.zeros(2)}, {}, 1 << 62)
    cases = [(len(header), 2 * 80, "do not match"),  # two descriptors for one tensor
             (len(header), 80 * 1025, "descriptor length"),
             (0, 80, "header length")]
    try:
        for size, described, _ in cases:
            if rank == 0:
                dist.send(torch.tensor([size, described], dtype=torch.int64), dst=1)
                if described == 2 * 80:
                    dist.send(torch.frombuffer(bytearray(header) + bytes(described), dtype=torch.uint8), dst=1)
            else:
                with pytest.raises(ValueError) as caught:
                    IpcChannel().recv(src=0)
                assert [m for s, d, m in cases if (s, d) == (size, described)][0] in str(caught.value)
    except Exception as error:
        failures.put((rank, repr(error)))
        raise
    finally:
        dist.destroy_process_group()


def test_ipc_channel_rejects_bad_control_messages(tmp_path):
    ctx = mp.get_context("spawn")
    failures = ctx.SimpleQueue()
    procs = [ctx.Process(target=_ipc_control_peer, args=(r, str(tmp_path / "rendezvous"), failures)) for r in (0, 1)]
    for p in procs:
        p.start()
    for p in procs:
        p.join(120)
    seen = []
    while not failures.empty():
        seen.append(failures.get())
    assert not seen, seen
    assert [p.exitcode for p in procs] == [0, 0]
