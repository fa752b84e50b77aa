"""Two processes on one GPU exchanging packets through IpcChannel: header over
Gloo, bytes read from the sender's device memory through an IPC mapping.

Checks bit-exact delivery of the reference's transport fixture values
(non-contiguous and constant layers, three dtypes, layer order [7, 2]) and of
random packed KV layers, zero-size tensors, the lifetime protocol (the
sender's packet survives until the reply) and header validation."""
import os
from datetime import timedelta
from pathlib import Path

import pytest
import torch
import torch.distributed as dist
import torch.multiprocessing as mp

pytestmark = pytest.mark.gpu


def _worker(rank, rendezvous):
    from hexgen2_amd.transport import IpcChannel, recv_data, recv_packet, send_data, send_packet
    torch.cuda.set_device(0)
    dist.init_process_group("gloo", rank=rank, world_size=2, init_method=Path(rendezvous).as_uri(),
                            timeout=timedelta(seconds=60))
    channel = IpcChannel()
    try:
        g = torch.Generator(device="cuda").manual_seed(5)
        for round_, dtype in enumerate((torch.float16, torch.bfloat16, torch.float32)):
            cache = {7: torch.arange(-24, 24).reshape(1, 4, 2, 2, 3).to(dtype)[..., ::2].cuda(),
                     2: torch.full((1, 3, 2, 1, 4), -1.25, dtype=dtype, device="cuda")}
            token = torch.tensor([42, 17], dtype=torch.long, device="cuda")
            big = torch.randn((3, 1000, 2, 8, 128), generator=g, device="cuda").to(dtype)
            # tensors sharing one allocation: one export, one mapping, several views
            stacked = torch.randn((4, 33, 2, 8), generator=g, device="cuda").to(dtype)
            raw = torch.arange(64, dtype=torch.uint8, device="cuda")
            shared = {f"l{i}": stacked[i] for i in range(4)}
            shared.update(mid=stacked[1, 5:9], words=raw[8:40].view(torch.int64), byte=raw[3:4])
            if rank == 0:
                send_data(token, cache, dst=1, channel=channel)
                send_packet({"big": big, "empty": torch.zeros((0, 5), device="cuda")}, {"round": round_}, dst=1,
                            channel=channel)
                send_packet(shared, {"shared": round_}, dst=1, channel=channel)
                # the peer checks the bytes against this copy sent by value
                dist.send(big.cpu(), dst=1)
                received, returned = recv_data(src=1, num_layers=2, channel=channel)
                assert received.tolist() == [42, 17] and list(returned) == [7, 2]
                for key in cache:
                    assert torch.equal(returned[key].cpu(), cache[key].cpu()), key
                del received, returned
            else:
                received, returned = recv_data(src=0, num_layers=2, channel=channel)
                tensors, meta = recv_packet(src=0, channel=channel)
                views, view_meta = recv_packet(src=0, channel=channel)
                assert view_meta == {"shared": round_} and list(views) == list(shared)
                for name, want in shared.items():
                    got = views[name]
                    assert got.is_cuda and got.dtype == want.dtype and got.shape == want.shape, name
                    assert torch.equal(got.cpu(), want.cpu()), name
                del views
                expect = torch.empty((3, 1000, 2, 8, 128), dtype=dtype)
                dist.recv(expect, src=0)
                assert meta == {"round": round_}
                assert tensors["empty"].shape == (0, 5) and tensors["empty"].is_cuda
                assert tensors["big"].is_cuda and tensors["big"].dtype == dtype
                assert torch.equal(tensors["big"].cpu().view(torch.uint8), expect.view(torch.uint8))
                # read the peer's bytes with a kernel of this process too
                assert torch.equal((tensors["big"].float() * 2).cpu(), expect.float() * 2)
                copy_token, copy_cache = received.clone(), {k: v.clone() for k, v in returned.items()}
                del received, returned, tensors
                send_data(copy_token, copy_cache, dst=0, channel=channel)
        dist.barrier()
    finally:
        dist.destroy_process_group()


def test_ipc_packets_between_two_processes_on_one_gpu(tmp_path):
    os.environ.setdefault("HSA_ENABLE_IPC_MODE_LEGACY", "0")
    mp.spawn(_worker, args=(str(tmp_path / "rendezvous"),), nprocs=2, join=True)


def test_ipc_rejects_host_tensors(device):
    from hexgen2_amd.transport import IpcChannel
    with pytest.raises(ValueError, match="device tensors"):
        IpcChannel().send({"x": torch.zeros(3)}, {}, dst=1)


def test_ipc_export_refuses_allocations_of_2_gib(device):
    """The C ABI itself refuses a handle for an allocation that another
    process could not map (2 GiB or more), before any mapping is tried."""
    import ctypes
    from hexgen2_amd import _lib
    lib = _lib.load()
    handle, off, size = _lib.IpcHandle(), ctypes.c_uint64(), ctypes.c_uint64()
    big = torch.empty(2 * 1024 ** 3, dtype=torch.uint8, device=device)
    rc = lib.hexkv_ipc_export(ctypes.c_void_p(big.data_ptr() + 4096), ctypes.byref(handle), ctypes.byref(off),
                              ctypes.byref(size))
    assert rc == _lib.HEXKV_ERANGE and b"below 2 GiB" in lib.hexkv_last_error()
    del big
    small = torch.empty(1 << 20, dtype=torch.uint8, device=device)
    rc = lib.hexkv_ipc_export(ctypes.c_void_p(small.data_ptr() + 256), ctypes.byref(handle), ctypes.byref(off),
                              ctypes.byref(size))
    assert rc == 0 and off.value >= 256 and size.value >= (1 << 20)


def test_handoff_bench_runs_and_delivers_bit_exact():
    """python -m hexgen2_amd.handoff_bench on the tiny workload: two rounds,
    each rank reports, and the decode rank's unpack from the peer's memory
    is bit-exact on the sampled sequence."""
    import json
    import subprocess
    import sys
    root = Path(__file__).resolve().parents[1]
    env = dict(os.environ, HSA_ENABLE_IPC_MODE_LEGACY="0")
    print("handoff_bench tiny-llama, 2 rounds", flush=True)
    result = subprocess.run([sys.executable, "-m", "hexgen2_amd.handoff_bench", "--workload", "tiny-llama",
                             "--rounds", "2"], cwd=root, env=env, capture_output=True, text=True, timeout=100)
    assert result.returncode == 0, result.stderr[-2000:]
    lines = [json.loads(l) for l in result.stdout.splitlines() if l.startswith("{")]
    decode = [l for l in lines if l["rank"] == 1]
    assert sorted(l["round"] for l in lines if l["rank"] == 0) == [0, 1]
    assert [l["round"] for l in decode] == [0, 1]
    assert all(l["sampled_sequence_bit_exact"] and l["handoff_ms"] > 0 for l in decode)
