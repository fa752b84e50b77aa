"""Self-describing tensor packets between the prefill and decode phases.

Same entry points, header format and validation as the pilot's transport
(hexgen2/transport.py:13-100): ``validate_header``, ``send_packet``,
``recv_packet``, ``send_data``, ``recv_data``.  Three carriers:

* ``DeviceChannel`` -- prefill and decode in one process on the same GPU:
  the header is encoded, size-checked and parsed exactly as on the wire, and
  the tensors are handed over in device memory (no copy, no host round
  trip).  The receiver gets the sender's (contiguous) tensors; the sender
  must not modify them after sending, which the pilot never does
  (run.py:146-177).
* ``IpcChannel`` -- prefill and decode in two processes on the same GPU:
  the header plus one IPC descriptor per tensor travel over
  ``torch.distributed`` (a host group, e.g. Gloo), the bytes stay where the
  sender's kernels wrote them and the receiver reads them through a mapping
  of the sender's allocation (``hexkv_ipc_*`` in libhexkv).
* ``torch.distributed`` -- when no channel is active, packets use the
  reference's wire protocol (int64 header length, UTF-8 JSON header, then one
  send per non-empty tensor in header order), so a peer running the
  reference transport interoperates.

A channel is selected per call (``channel=``) or for a block of code
(``with use_channel(endpoint):``).
"""
from __future__ import annotations

import collections
import contextlib
import ctypes
import json
import math
import struct
import threading
from typing import Optional, Union

import torch
import torch.distributed as dist

DTYPES = {str(dtype): dtype for dtype in (
    torch.float16, torch.bfloat16, torch.float32, torch.float64,
    torch.int64, torch.int32, torch.int16, torch.int8, torch.uint8, torch.bool,
)}
MAX_HEADER = 1024 * 1024
MAX_PAYLOAD = 8 * 1024 ** 3
MAX_TENSORS = 1024
MAX_DIMS = 8

_ELEMENT_BYTES = {name: torch.empty((), dtype=dtype).element_size() for name, dtype in DTYPES.items()}


def validate_header(header, max_payload: int = MAX_PAYLOAD) -> int:
    """Check a decoded packet header; returns its payload bytes.

    Rejects (ValueError) what hexgen2/transport.py:25-41 rejects: a version
    other than 1, a missing tensor list, more than 1024 tensors, duplicate or
    non-string names, unknown dtypes, shapes that are not lists of at most 8
    non-negative ints (bools are not ints here), and payloads above
    ``max_payload`` (8 GiB on the wire).
    """
    if header.get("version") != 1 or not isinstance(header.get("tensors"), list):
        raise ValueError("Unsupported tensor packet")
    if len(header["tensors"]) > MAX_TENSORS:
        raise ValueError("Too many tensors")
    size, names = 0, set()
    for item in header["tensors"]:
        name, shape, dtype = item["name"], item["shape"], item["dtype"]
        if not isinstance(name, str) or name in names or dtype not in DTYPES:
            raise ValueError("Invalid tensor name or dtype")
        if not isinstance(shape, list) or len(shape) > MAX_DIMS or any(
                type(d) is not int or d < 0 for d in shape):
            raise ValueError("Invalid tensor shape")
        size += math.prod(shape) * _ELEMENT_BYTES[dtype]
        names.add(name)
    if size > max_payload:
        raise ValueError("Tensor packet exceeds memory limit")
    return size


def _encode_header(tensors, metadata, max_payload):
    header = {"version": 1, "metadata": metadata, "tensors": [
        {"name": name, "shape": list(t.shape), "dtype": str(t.dtype)} for name, t in tensors.items()
    ]}
    payload_bytes = validate_header(header, max_payload)
    encoded = json.dumps(header, allow_nan=False).encode("utf-8")
    if not 0 < len(encoded) <= MAX_HEADER:
        raise ValueError("Tensor metadata exceeds limit")
    return encoded, payload_bytes


def _decode_header(encoded: bytes, max_payload):
    if not 0 < len(encoded) <= MAX_HEADER:
        raise ValueError("Invalid tensor header length")
    header = json.loads(encoded.decode("utf-8"))
    validate_header(header, max_payload)
    return header


class DeviceChannel:
    """One endpoint of an in-process, same-GPU packet channel.

    ``a, b = DeviceChannel.pair()`` gives ranks 0 and 1; ``a`` sends to
    ``dst=1`` and receives from ``src=1``.  Packets queue in order per
    (src, dst).  ``max_payload`` bounds a packet (default: no bound beyond
    device memory, since nothing is copied; the wire limit is 8 GiB).
    """

    def __init__(self, rank: int, mailboxes: dict, lock: threading.Lock,
                 max_payload: Optional[int] = None):
        self.rank = rank
        self._mailboxes = mailboxes
        self._lock = lock
        self.max_payload = max_payload if max_payload is not None else 1 << 62

    @classmethod
    def pair(cls, max_payload: Optional[int] = None):
        mailboxes = collections.defaultdict(collections.deque)
        lock = threading.Lock()
        return cls(0, mailboxes, lock, max_payload), cls(1, mailboxes, lock, max_payload)

    def send(self, tensors, metadata, dst: int) -> int:
        encoded, payload = _encode_header(tensors, metadata, self.max_payload)
        items = [tensor.detach().contiguous() for tensor in tensors.values()]
        with self._lock:
            self._mailboxes[(self.rank, dst)].append((encoded, items))
        return payload

    def recv(self, src: int):
        with self._lock:
            box = self._mailboxes[(src, self.rank)]
            if not box:
                raise RuntimeError(f"no packet from rank {src} is waiting for rank {self.rank}")
            encoded, items = box.popleft()
        header = _decode_header(encoded, self.max_payload)
        tensors = {}
        for item, tensor in zip(header["tensors"], items):
            if list(tensor.shape) != item["shape"] or str(tensor.dtype) != item["dtype"]:
                raise ValueError("Packet tensor does not match its header")
            tensors[item["name"]] = tensor
        return tensors, header["metadata"]


# DLPack (v0.8) type codes of the packet dtypes: (code, bits).
_DLPACK = {torch.float16: (2, 16), torch.bfloat16: (4, 16), torch.float32: (2, 32),
           torch.float64: (2, 64), torch.int64: (0, 64), torch.int32: (0, 32),
           torch.int16: (0, 16), torch.int8: (0, 8), torch.uint8: (1, 8), torch.bool: (6, 8)}
_DESCRIPTOR = struct.Struct("<64sQQ")  # IPC handle, byte offset in the allocation, allocation bytes
IPC_ALLOCATION_LIMIT = 2 * 1024 ** 3  # mapped allocations must stay below 2 GiB on this platform
_CAPSULE_NAME = b"dltensor"
_capsule_new = ctypes.pythonapi.PyCapsule_New
_capsule_new.restype = ctypes.py_object
_capsule_new.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p]


class IpcChannel:
    """Packets between two processes that share one GPU.

    ``send`` encodes and validates the header exactly as the wire does, makes
    every tensor contiguous on the device, synchronises the sender's stream so
    the bytes are complete, and sends over ``torch.distributed`` (``group``;
    host tensors only): the header's and the descriptors' lengths (int64),
    then one message of the header followed by one 80-byte descriptor per
    tensor (IPC handle of the allocation holding it, byte offset, allocation
    size).  ``recv`` maps each allocation once and
    returns tensors that alias the sender's memory, views of one byte tensor
    over the mapping (zero-size tensors are created locally).  Tensors of one
    packet that share an allocation (the layers of one packed buffer) cost
    one handle export and one mapping, not one each: an export takes ~9 us
    of host time on MI355X.

    Lifetime protocol: the sender keeps every tensor of a packet alive until
    it next receives a packet from that peer; the receiver must drop the
    tensors of a packet (which unmaps them) before it sends to that peer
    again.  The prefill/decode request cycle (send KV, reply with tokens)
    follows it.
    """

    def __init__(self, group=None, max_payload: Optional[int] = None):
        self.group = group
        self.max_payload = max_payload if max_payload is not None else 1 << 62
        self._held = collections.defaultdict(list)

    def send(self, tensors, metadata, dst: int) -> int:
        from . import _lib
        encoded, payload = _encode_header(tensors, metadata, self.max_payload)
        lib = _lib.load()
        items, descriptors = [], bytearray()
        exported = {}  # storage address -> (handle, storage's offset in its allocation, allocation bytes)
        for name, tensor in tensors.items():
            tensor = tensor.detach()
            if not tensor.is_cuda:
                raise ValueError(f"IPC packets carry device tensors; {name!r} is on {tensor.device}")
            tensor = tensor.contiguous()
            items.append(tensor)
            if tensor.numel() == 0:
                descriptors += _DESCRIPTOR.pack(bytes(64), 0, 0)
                continue
            storage = tensor.untyped_storage().data_ptr()
            entry = exported.get(storage)
            if entry is None:
                handle, offset, size = _lib.IpcHandle(), ctypes.c_uint64(), ctypes.c_uint64()
                _lib.check(lib.hexkv_ipc_export(storage, ctypes.byref(handle), ctypes.byref(offset),
                                                ctypes.byref(size)), "hexkv_ipc_export")
                if size.value >= IPC_ALLOCATION_LIMIT:
                    raise ValueError(f"tensor {name!r} lives in a {size.value}-byte allocation; IPC handoff "
                                     "needs allocations below 2 GiB (send it in per-layer tensors)")
                entry = exported[storage] = (bytes(handle.bytes), offset.value, size.value)
            handle_bytes, storage_offset, alloc = entry
            descriptors += _DESCRIPTOR.pack(handle_bytes, storage_offset + (tensor.data_ptr() - storage), alloc)
        torch.cuda.current_stream().synchronize()
        dist.send(torch.tensor([len(encoded), len(descriptors)], dtype=torch.int64), dst=dst, group=self.group)
        dist.send(torch.frombuffer(bytearray(encoded) + descriptors, dtype=torch.uint8), dst=dst, group=self.group)
        self._held[dst].append(items)
        return payload

    def recv(self, src: int):
        from . import _lib
        self._held[src].clear()  # the peer has dropped our earlier packets
        lengths = torch.empty(2, dtype=torch.int64)
        dist.recv(lengths, src=src, group=self.group)
        size, described = (int(n) for n in lengths.tolist())
        if not 0 < size <= MAX_HEADER:
            raise ValueError("Invalid tensor header length")
        if not 0 <= described <= _DESCRIPTOR.size * MAX_TENSORS:
            raise ValueError("Invalid IPC descriptor length")
        message = torch.empty(size + described, dtype=torch.uint8)
        dist.recv(message, src=src, group=self.group)
        data = message.numpy().tobytes()
        header = _decode_header(data[:size], self.max_payload)
        if described != _DESCRIPTOR.size * len(header["tensors"]):
            raise ValueError("IPC descriptors do not match the header's tensors")
        raw = data[size:]
        lib = _lib.load()
        device = torch.cuda.current_device()
        tensors, mapped = {}, {}  # mapped: handle -> (uint8 tensor over the whole allocation)
        for i, item in enumerate(header["tensors"]):
            handle_bytes, offset, alloc = _DESCRIPTOR.unpack_from(raw, i * _DESCRIPTOR.size)
            dtype, shape = DTYPES[item["dtype"]], item["shape"]
            elem = _ELEMENT_BYTES[item["dtype"]]
            nbytes = math.prod(shape) * elem
            if nbytes == 0:
                tensors[item["name"]] = torch.empty(shape, dtype=dtype, device=device)
                continue
            if offset + nbytes > alloc or offset % elem:
                raise ValueError("IPC descriptor does not cover the tensor its header names")
            whole = mapped.get((handle_bytes, alloc))
            if whole is None:
                handle = _lib.IpcHandle()
                ctypes.memmove(handle.bytes, handle_bytes, 64)
                base = ctypes.c_void_p()
                _lib.check(lib.hexkv_ipc_open(ctypes.byref(handle), ctypes.byref(base)), "hexkv_ipc_open")
                code, bits = _DLPACK[torch.uint8]
                managed = lib.hexkv_ipc_dlpack(base, 0, 1, (ctypes.c_int64 * 1)(alloc), code, bits, device)
                if not managed:
                    lib.hexkv_ipc_close(base)
                    raise ValueError(lib.hexkv_last_error().decode())
                # the mapping is released when this tensor and every view of it are gone
                whole = mapped[(handle_bytes, alloc)] = torch.utils.dlpack.from_dlpack(
                    _capsule_new(managed, _CAPSULE_NAME, None))
            tensors[item["name"]] = whole[offset:offset + nbytes].view(dtype).view(shape)
        return tensors, header["metadata"]


_active = threading.local()


Channel = Union[DeviceChannel, IpcChannel]


@contextlib.contextmanager
def use_channel(channel: Channel):
    """Route send_packet/recv_packet calls in this block through ``channel``."""
    previous = getattr(_active, "channel", None)
    _active.channel = channel
    try:
        yield channel
    finally:
        _active.channel = previous


def _channel(channel):
    return channel if channel is not None else getattr(_active, "channel", None)


def wire_device():
    """Device of wire tensors: the current GPU for NCCL/RCCL, else the CPU."""
    return (torch.device("cuda", torch.cuda.current_device()) if dist.get_backend() == "nccl"
            else torch.device("cpu"))


def send_packet(tensors, metadata, dst, channel: Optional[Channel] = None):
    """Send named tensors plus JSON metadata to ``dst``; returns payload bytes."""
    channel = _channel(channel)
    if channel is not None:
        return channel.send(tensors, metadata, dst)
    encoded, payload_bytes = _encode_header(tensors, metadata, MAX_PAYLOAD)
    device = wire_device()
    dist.send(torch.tensor([len(encoded)], dtype=torch.int64, device=device), dst=dst)
    dist.send(torch.frombuffer(bytearray(encoded), dtype=torch.uint8).to(device), dst=dst)
    for tensor in tensors.values():
        tensor = tensor.detach().to(device).contiguous()
        if tensor.numel():
            dist.send(tensor, dst=dst)
    return payload_bytes


def recv_packet(src, channel: Optional[Channel] = None):
    """Receive one packet from ``src``; returns (dict of tensors, metadata)."""
    channel = _channel(channel)
    if channel is not None:
        return channel.recv(src)
    device = wire_device()
    length = torch.empty(1, dtype=torch.int64, device=device)
    dist.recv(length, src=src)
    size = int(length.item())
    if not 0 < size <= MAX_HEADER:
        raise ValueError("Invalid tensor header length")
    encoded = torch.empty(size, dtype=torch.uint8, device=device)
    dist.recv(encoded, src=src)
    header = _decode_header(bytes(encoded.cpu().numpy().tobytes()), MAX_PAYLOAD)
    tensors = {}
    for item in header["tensors"]:
        tensor = torch.empty(item["shape"], dtype=DTYPES[item["dtype"]], device=device)
        if tensor.numel():
            dist.recv(tensor, src=src)
        tensors[item["name"]] = tensor
    return tensors, header["metadata"]


def send_data(single_tensor, tensor_dict, dst, channel: Optional[Channel] = None):
    """Legacy API: a token tensor plus a KV dict keyed by int layer
    (hexgen2/transport.py:83-90)."""
    keys = list(tensor_dict)
    if any(type(key) is not int for key in keys):
        raise ValueError("KV-cache layer keys must be integers")
    return send_packet({"token": single_tensor, **{f"kv/{key}": tensor_dict[key] for key in keys}},
                       {"layers": keys}, dst, channel=channel)


def recv_data(src, num_layers=None, tensor_shape=None, channel: Optional[Channel] = None):
    """Legacy API counterpart of ``send_data`` (hexgen2/transport.py:93-100)."""
    tensors, metadata = recv_packet(src, channel=channel)
    cache = {key: tensors[f"kv/{key}"] for key in metadata["layers"]}
    if num_layers is not None and len(cache) != num_layers:
        raise ValueError("Received KV-cache layer count differs from expected count")
    if tensor_shape is not None and any(tuple(t.shape) != tuple(tensor_shape) for t in cache.values()):
        raise ValueError("Received KV-cache shape differs from expected shape")
    return tensors["token"], cache
