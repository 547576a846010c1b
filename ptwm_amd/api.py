"""Python entry points mirroring the reference's PyO3 device API.

Same names, argument meaning and error behaviour as
``crates/ptwm-py/src/plane_codec_cuda.rs:74-190`` and
``crates/ptwm-py/src/hardware.rs:55-154``, backed by libptwm_mi355x.so:

- ``plane_codec_encode_cuda(selector, codec_id, state_bytes, src, dst, device_ordinal)``
- ``plane_codec_decode_cuda(selector, codec_id, state_bytes, src, dst, device_ordinal)``
- ``hardware_backend_cuda_stream_handle(canonical_id, device_ordinal)``
- ``hardware_backend_dispatch_decode_cuda(canonical_id, codec_id, state_bytes, compressed, out, device_ordinal)``

``src``/``dst`` are contiguous ``torch.Tensor`` objects resident on the
device.  As in the reference, which exports each tensor with
``__dlpack__(stream=<library stream>)``, work pending on the producer's
stream is ordered before the library's stream touches the memory (for torch
tensors with one event, see ``_order_after_producer``); the device ordinal
of every tensor must equal ``device_ordinal`` (plane_codec_cuda.rs:120-124).
"""
from __future__ import annotations

import ctypes as C
import threading

from . import ids
from . import _native
from ._native import RC_BUFFER_TOO_SMALL, NativeError, check, lib


def _current_raw_stream(device_ordinal: int) -> int:
    import torch
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is not None:
        return int(raw(device_ordinal))
    return int(torch.cuda.current_stream(device_ordinal).cuda_stream)


_tls = threading.local()   # per thread: device -> stream the library was asked to run on


def _use_stream(device_ordinal: int, s) -> None:
    """Ask the library to run this thread's calls on stream s (None: its own)."""
    used = getattr(_tls, "used", None)
    if used is None:
        used = _tls.used = {}
    if used.get(device_ordinal, "own") == s:
        return
    check(lib().ptwm_mi355x_use_stream(0 if s is None else s, 0 if s is None else 1, device_ordinal),
          "stream selection")
    used[device_ordinal] = s


def _order_after_producer(t, device_ordinal: int, stream: int) -> None:
    """Stream-ordered hand-off, as the reference's ``__dlpack__(stream=...)``:
    work already queued on the producer's current stream completes before
    the library touches the memory.  For torch tensors the library runs this
    thread's calls on torch's current stream (``ptwm_mi355x_use_stream``), so
    no event is needed; any other DLPack object goes through ``__dlpack__``
    with the library's own stream."""
    import torch
    if not isinstance(t, torch.Tensor):
        _use_stream(device_ordinal, None)
        t.__dlpack__(stream=stream)
        return
    _use_stream(device_ordinal, _current_raw_stream(device_ordinal))


def _both_torch(a, b) -> bool:
    """One ordering event covers both tensors when both are torch tensors
    (they share torch's current stream)."""
    return type(a).__module__.startswith("torch") and type(b).__module__.startswith("torch")


def _dev_ptr_len(t, name: str, device_ordinal: int, stream: int, writable: bool, ordered: bool = False):
    if not hasattr(t, "__dlpack__") or not hasattr(t, "data_ptr"):
        raise TypeError(f"{name}: expected a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name}: tensor must be contiguous")
    if not t.is_cuda:
        raise ValueError(f"{name}: tensor is not on a GPU device")
    dev = t.get_device()
    if dev != device_ordinal:
        raise ValueError(f"{name}: tensor is on device {dev}, call names device {device_ordinal}")
    if not ordered:
        _order_after_producer(t, device_ordinal, stream)
    return int(t.data_ptr()), int(t.nbytes)


def _resolve_own(selector: str, label: str) -> None:
    got = ids.resolve_codec_selector(selector)
    if got != _own_id(label):
        raise LookupError(f"selector {selector!r} does not name this library's {label}")


def _own_id(label: str) -> bytes:
    c = _OWN_BYTES.get(label)
    if c is None:
        c = _OWN_BYTES[label] = bytes.fromhex(ids.OWN_IDS[label])
    return c


_OWN_BYTES: dict = {}


def plane_codec_decode_cuda(selector: str, codec_id: str, state_bytes: bytes, src, dst,
                            device_ordinal: int, policy=None) -> int:
    _resolve_own(selector, ids.PLANE_CODEC_LABEL)
    codec = ids.resolve_codec_selector(codec_id)
    L = lib()
    stream = int(L.ptwm_plane_codec_v1_cuda_stream_handle(device_ordinal))
    if stream == 0:
        raise NativeError(-5, "plane_codec_decode_cuda: no stream for device")
    ip, il = _dev_ptr_len(src, "src", device_ordinal, stream, False)
    op, ol = _dev_ptr_len(dst, "dst", device_ordinal, stream, True, _both_torch(src, dst))
    st = bytes(state_bytes)
    rc = L.ptwm_plane_codec_v1_decode_cuda(1, st if st else None, len(st), codec, 32, ip, il, op, ol,
                                           device_ordinal)
    return check(rc, "plane_codec_decode_cuda")


def plane_codec_encode_cuda(selector: str, codec_id: str, state_bytes: bytes, src, dst,
                            device_ordinal: int, policy=None) -> int:
    _resolve_own(selector, ids.PLANE_CODEC_LABEL)
    codec = ids.resolve_codec_selector(codec_id)
    L = lib()
    stream = int(L.ptwm_plane_codec_v1_cuda_stream_handle(device_ordinal))
    if stream == 0:
        raise NativeError(-5, "plane_codec_encode_cuda: no stream for device")
    ip, il = _dev_ptr_len(src, "src", device_ordinal, stream, False)
    op, ol = _dev_ptr_len(dst, "dst", device_ordinal, stream, True, _both_torch(src, dst))
    st = bytes(state_bytes)
    needed = C.c_uint64(0)
    rc = L.ptwm_plane_codec_v1_encode_cuda(1, st if st else None, len(st), codec, 32, ip, il, op, ol,
                                           C.byref(needed), device_ordinal)
    if rc == -2:
        err = NativeError(rc, f"plane_codec_encode_cuda: needs {needed.value} bytes")
        err.needed = needed.value
        raise err
    return check(rc, "plane_codec_encode_cuda")


def hardware_backend_cuda_stream_handle(canonical_id: str, device_ordinal: int, policy=None) -> int:
    _resolve_own(canonical_id, ids.HARDWARE_BACKEND_LABEL)
    h = int(lib().ptwm_hardware_backend_v1_cuda_stream_handle(device_ordinal))
    if h == 0:
        raise NativeError(-5, "hardware backend failed to produce a stream handle")
    return h


def hardware_backend_dispatch_decode_cuda(canonical_id: str, codec_id: str, state_bytes: bytes, compressed, out,
                                          device_ordinal: int, policy=None) -> int:
    stream = hardware_backend_cuda_stream_handle(canonical_id, device_ordinal)
    codec = ids.resolve_codec_selector(codec_id)
    ip, il = _dev_ptr_len(compressed, "compressed", device_ordinal, stream, False)
    op, ol = _dev_ptr_len(out, "out", device_ordinal, stream, True, _both_torch(compressed, out))
    st = state_bytes if isinstance(state_bytes, bytes) else bytes(state_bytes)
    rc = lib().ptwm_hardware_backend_v1_dispatch_decode_cuda(1, st if st else None, len(st), codec, 32, ip, il, op,
                                                             ol, device_ordinal)
    return check(rc, "hardware_backend_dispatch_decode_cuda")


def encode_tensor_cuda(chain: int, src, out, device_ordinal: int = 0, codec: str = "huff_ilv") -> tuple[int, bytes]:
    """Tensor-level GPU encode (library addition): split by ``chain``, code
    every plane with this library's GPU-native codec ``codec`` ("huff_ilv"
    or "rans_ilv"; Identity when coding does not shrink a plane).  Returns
    (bytes used in ``out``, PTMD decode plan)."""
    L = lib()
    fn = {"huff_ilv": L.ptwm_mi355x_encode_tensor_cuda, "rans_ilv": L.ptwm_mi355x_encode_tensor_rans_cuda}[codec]
    stream = int(L.ptwm_plane_codec_v1_cuda_stream_handle(device_ordinal))
    ip, il = _dev_ptr_len(src, "src", device_ordinal, stream, False)
    op, ol = _dev_ptr_len(out, "out", device_ordinal, stream, True)
    plan_buf = (C.c_uint8 * 4096)()
    plan_len = C.c_size_t(0)
    needed = C.c_uint64(0)
    rc = fn(chain, ip, il, op, ol, plan_buf, 4096, C.byref(plan_len), C.byref(needed), device_ordinal)
    if rc == -2:
        err = NativeError(rc, f"encode_tensor_cuda: needs {needed.value} bytes")
        err.needed = needed.value
        raise err
    check(rc, "encode_tensor_cuda")
    return rc, bytes(plan_buf[: plan_len.value])


def encode_tensors_cuda(items, out, device_ordinal: int = 0, codec: str = "huff_ilv") -> tuple[int, bytes]:
    """Tensor-level GPU encode of many tensors in one call (library
    addition): ``items`` is a sequence of (chain, device tensor); every plane
    coded with ``codec`` ("huff_ilv" or "rans_ilv"), batches of about 4 GiB
    of input through one encoder pass each.  Returns (bytes used in ``out``,
    one PTMD plan whose tensors are restored back to back at 256-byte
    aligned offsets in the given order)."""
    L = lib()
    fam = {"huff_ilv": 0, "rans_ilv": 1}[codec]
    stream = int(L.ptwm_plane_codec_v1_cuda_stream_handle(device_ordinal))
    items = list(items)
    n = len(items)
    chains = (C.c_uint32 * max(n, 1))()
    ptrs = (C.c_uint64 * max(n, 1))()
    lens = (C.c_uint64 * max(n, 1))()
    for i, (chain, src) in enumerate(items):
        ip, il = _dev_ptr_len(src, "src", device_ordinal, stream, False, i > 0)
        chains[i], ptrs[i], lens[i] = chain, ip, il
    op, ol = _dev_ptr_len(out, "out", device_ordinal, stream, True, True)
    cap = 12 + sum(20 + 32 * 4 for _ in range(n))
    plan_buf = (C.c_uint8 * cap)()
    plan_len = C.c_size_t(0)
    needed = C.c_uint64(0)
    rc = L.ptwm_mi355x_encode_tensors_cuda(fam, n, chains, ptrs, lens, op, ol, plan_buf, cap, C.byref(plan_len),
                                           C.byref(needed), device_ordinal)
    if rc == -2:
        err = NativeError(rc, f"encode_tensors_cuda: needs {needed.value} bytes")
        err.needed = needed.value
        raise err
    check(rc, "encode_tensors_cuda")
    return rc, bytes(plan_buf[: plan_len.value])


CODEC_SELECT = 0xFFFF  # PTWM_MI355X_CODEC_SELECT: trial-encode selection


def encode_tensor_ref_cuda(chain: int, plane_codecs, chunk_size: int, src, out,
                           device_ordinal: int = 0) -> tuple[int, bytes]:
    """Tensor-level GPU encode into the reference's plane formats (library
    addition): split by ``chain``; plane p coded with ``plane_codecs[p]``
    (wire ids 0 Identity, 1 Huffman, 3 rANS, or CODEC_SELECT: the
    reference's trial encode picks one), chunked at ``chunk_size`` bytes (0:
    one payload per plane).  Returns (bytes used in ``out``, PTMD decode
    plan)."""
    L = lib()
    stream = int(L.ptwm_plane_codec_v1_cuda_stream_handle(device_ordinal))
    ip, il = _dev_ptr_len(src, "src", device_ordinal, stream, False)
    op, ol = _dev_ptr_len(out, "out", device_ordinal, stream, True, _both_torch(src, out))
    codecs = (C.c_uint16 * len(plane_codecs))(*plane_codecs)
    plan_len = C.c_size_t(0)
    needed = C.c_uint64(0)
    cap = 4096
    while True:
        plan_buf = (C.c_uint8 * cap)()
        rc = L.ptwm_mi355x_encode_tensor_ref_cuda(chain, codecs, len(plane_codecs), chunk_size, ip, il, op, ol,
                                                  plan_buf, cap, C.byref(plan_len), C.byref(needed), device_ordinal)
        if rc == -2 and plan_len.value > cap:
            cap = plan_len.value
            continue
        break
    if rc == -2:
        err = NativeError(rc, f"encode_tensor_ref_cuda: needs {needed.value} bytes")
        err.needed = needed.value
        raise err
    check(rc, "encode_tensor_ref_cuda")
    return rc, bytes(plan_buf[: plan_len.value])


PLANE_OP_INT_DELTA = 1
PLANE_OP_PREDICTOR_XOR = 2
PLANE_OP_MANTISSA_ZERO_STRIP = 3


def plane_op_spec(op: int, param: int) -> int:
    """An encoder plane-op spec: op | param << 8 (0: none)."""
    return 0 if op == 0 else op | param << 8


def encode_tensor_ref_ops_cuda(chain: int, plane_codecs, plane_ops, chunk_size: int, src, out,
                               device_ordinal: int = 0, chain_trial: bool = False) -> tuple[int, bytes, list[int]]:
    """As :func:`encode_tensor_ref_cuda`, each plane first passed through its
    op (``plane_ops[p]``: :func:`plane_op_spec`), or with ``chain_trial`` the
    reference's trial among the production split-chain variants (library
    addition).  Returns (bytes used in ``out``, PTMD plan, chosen op specs)."""
    L = lib()
    stream = int(L.ptwm_plane_codec_v1_cuda_stream_handle(device_ordinal))
    ip, il = _dev_ptr_len(src, "src", device_ordinal, stream, False)
    op, ol = _dev_ptr_len(out, "out", device_ordinal, stream, True, _both_torch(src, out))
    n = len(plane_codecs)
    codecs = (C.c_uint16 * n)(*plane_codecs)
    ops = (C.c_uint16 * n)(*(plane_ops if plane_ops is not None else [0] * n))
    ops_out = (C.c_uint16 * n)()
    plan_len = C.c_size_t(0)
    needed = C.c_uint64(0)
    cap = 4096
    while True:
        plan_buf = (C.c_uint8 * cap)()
        rc = L.ptwm_mi355x_encode_tensor_ref_ops_cuda(chain, codecs, ops, n, 1 if chain_trial else 0, chunk_size,
                                                      ip, il, op, ol, plan_buf, cap, C.byref(plan_len),
                                                      C.byref(needed), ops_out, device_ordinal)
        if rc == -2 and plan_len.value > cap:
            cap = plan_len.value
            continue
        break
    if rc == -2:
        err = NativeError(rc, f"encode_tensor_ref_ops_cuda: needs {needed.value} bytes")
        err.needed = needed.value
        raise err
    check(rc, "encode_tensor_ref_ops_cuda")
    return rc, bytes(plan_buf[: plan_len.value]), list(ops_out)


def plane_crc32_cuda(chain: int, src, device_ordinal: int = 0) -> list[int]:
    """CRC-32 (crc32fast::hash) of every plane of the device tensor ``src``
    split by ``chain`` (library addition; the per-plane checksum of
    container.rs:2154-2159)."""
    L = lib()
    stream = int(L.ptwm_plane_codec_v1_cuda_stream_handle(device_ordinal))
    ip, il = _dev_ptr_len(src, "src", device_ordinal, stream, False)
    out = (C.c_uint32 * 4)()
    n = check(L.ptwm_mi355x_plane_crc32_cuda(chain, ip, il, out, 4, device_ordinal), "plane_crc32_cuda")
    return [int(out[i]) for i in range(n)]


def decode_stats(device_ordinal: int = 0) -> dict:
    """Cumulative path counts of the device's reference-format Huffman
    payloads (library addition): accepted by the parallel decode, decoded
    again by the exact state machine, calls that needed extra fix passes."""
    out = (C.c_uint64 * 3)()
    check(lib().ptwm_mi355x_decode_stats(device_ordinal, out, 3), "decode_stats")
    return {"accepted": int(out[0]), "fallbacks": int(out[1]), "extra_rounds": int(out[2])}


def xxh64_cuda(src, device_ordinal: int = 0) -> int:
    """XXH64 (seed 0) of the device bytes ``src`` (library addition; the
    tensor payload hash of container.rs:2185-2194)."""
    L = lib()
    stream = int(L.ptwm_plane_codec_v1_cuda_stream_handle(device_ordinal))
    ip, il = _dev_ptr_len(src, "src", device_ordinal, stream, False)
    h = C.c_uint64(0)
    check(L.ptwm_mi355x_xxh64_cuda(ip, il, C.byref(h), device_ordinal), "xxh64_cuda")
    return int(h.value)


def split_cuda(chain: int, src, planes, device_ordinal: int = 0) -> int:
    """Forward chain on device (library addition)."""
    L = lib()
    stream = int(L.ptwm_plane_codec_v1_cuda_stream_handle(device_ordinal))
    ip, il = _dev_ptr_len(src, "src", device_ordinal, stream, False)
    arr = (C.c_uint64 * len(planes))(*[_dev_ptr_len(p, "plane", device_ordinal, stream, True)[0] for p in planes])
    return check(L.ptwm_mi355x_split_cuda(chain, ip, il, arr, len(planes), device_ordinal), "split_cuda")


def merge_cuda(chain: int, planes, out, device_ordinal: int = 0) -> int:
    """Inverse chain on device (library addition)."""
    L = lib()
    stream = int(L.ptwm_plane_codec_v1_cuda_stream_handle(device_ordinal))
    ptrs = [_dev_ptr_len(p, "plane", device_ordinal, stream, False) for p in planes]
    op, ol = _dev_ptr_len(out, "out", device_ordinal, stream, True)
    arr = (C.c_uint64 * len(planes))(*[p[0] for p in ptrs])
    return check(L.ptwm_mi355x_merge_cuda(chain, arr, len(planes), ptrs[0][1], op, ol, device_ordinal), "merge_cuda")


class ContainerEntry:
    """One tensor of a container as ``container_plan`` lists it."""

    __slots__ = ("name", "orig_size", "out_offset", "record_offset", "record_len", "dtype_code", "input_format",
                 "chain", "status", "plan_index", "hash_checked", "crc_checked")

    def __init__(self, t, data: bytes):
        # a record the reader rejected (status -1) may hold a malformed name
        self.name = bytes(data[t.name_offset:t.name_offset + t.name_len]).decode("utf-8", errors="replace")
        self.orig_size = int(t.orig_size)
        self.out_offset = int(t.out_offset)
        self.record_offset = int(t.record_offset)
        self.record_len = int(t.record_len)
        self.dtype_code = int(t.dtype_code)
        self.input_format = int(t.input_format)
        self.chain = int(t.chain)
        self.status = int(t.status)
        self.plan_index = int(t.plan_index)
        self.hash_checked = bool(t.flags & 1)
        self.crc_checked = bool(t.flags & 2)

    def __repr__(self):
        return (f"ContainerEntry({self.name!r}, orig_size={self.orig_size}, chain={self.chain}, "
                f"status={self.status}, out_offset={self.out_offset})")


def _host_buf(data):
    """(pointer argument, length, object to keep alive) of host bytes
    (bytes, bytearray, memoryview or a numpy array), without a copy."""
    if isinstance(data, bytes):
        return data, len(data), data
    import numpy as np

    a = data.reshape(-1).view(np.uint8) if isinstance(data, np.ndarray) else np.frombuffer(data, np.uint8)
    a = np.ascontiguousarray(a)
    return C.c_void_p(int(a.ctypes.data) if a.size else None), int(a.size), a


def container_plan(data) -> tuple[bytes, list[ContainerEntry], int]:
    """Read a .ptwm container (legacy or PTWC) or a PTWS frame held in host
    memory (bytes or a numpy uint8 array; library addition: the
    reference-side plan construction of container.rs:1590-1892 /
    compact.rs:407-480).  Returns the PTMD plan whose payload offsets index
    ``data``, the tensors in record order, and the output buffer length the
    plan restores into."""
    ptr, size, buf = _host_buf(data)
    L = lib()
    plan_len, n_t, out_len = C.c_size_t(0), C.c_size_t(0), C.c_uint64(0)
    rc = L.ptwm_mi355x_container_plan(ptr, size, None, 0, C.byref(plan_len), None, 0, C.byref(n_t),
                                      C.byref(out_len))
    if rc != RC_BUFFER_TOO_SMALL and rc < 0:
        check(rc, "container_plan")
    plan = (C.c_uint8 * max(plan_len.value, 1))()
    arr = (_native.ContainerTensor * max(n_t.value, 1))()
    rc = L.ptwm_mi355x_container_plan(ptr, size, plan, plan_len.value, C.byref(plan_len), arr, n_t.value,
                                      C.byref(n_t), C.byref(out_len))
    check(rc, "container_plan")
    entries = [ContainerEntry(arr[i], buf) for i in range(n_t.value)]
    return bytes(plan[:plan_len.value]), entries, int(out_len.value)


def container_rewrite(data) -> bytes:
    """Read a compact container (\\x89PTWC) or frame (\\x89PTWS) into its
    sections and records and write it again through the library's writer
    (library addition: the writers of ptwc.rs, tensor_record_compact.rs,
    chain/wire_compact.rs and compact.rs).  A file the reference wrote comes
    back byte for byte."""
    buf = bytes(data)
    L = lib()
    n = C.c_size_t(0)
    rc = L.ptwm_mi355x_container_rewrite(buf, len(buf), None, 0, C.byref(n))
    if rc != RC_BUFFER_TOO_SMALL and rc < 0:
        check(rc, "container_rewrite")
    out = (C.c_uint8 * max(n.value, 1))()
    check(L.ptwm_mi355x_container_rewrite(buf, len(buf), out, n.value, C.byref(n)), "container_rewrite")
    return bytes(out[:n.value])


class WritePlane:
    """One encoded plane for ``container_write``: codec wire id, payload
    (host bytes, or an (offset, length) span of the ``payloads`` buffer
    given to ``container_write``), optional CRC-32 of the plane and chunk
    table [(offset, size)]."""

    def __init__(self, codec: int, payload, crc32=None, chunks=None):
        self.codec, self.crc32, self.chunks = codec, crc32, chunks
        self.payload = tuple(int(v) for v in payload) if isinstance(payload, tuple) else bytes(payload)


class WriteTensor:
    """One tensor for ``container_write``: name, public dtype code
    (dtype.rs:79-103), decode-plan chain (plan.CHAIN_*), shape, planes in
    the chain's plane order, optional XXH64 of the tensor's bytes."""

    def __init__(self, name: str, dtype_code: int, chain: int, shape, planes, xxh64=None, input_format: int = 2):
        self.name, self.dtype_code, self.chain, self.shape = name, dtype_code, chain, list(shape)
        self.planes, self.xxh64, self.input_format = planes, xxh64, input_format


def container_write(tensors, layout: str = "compact", payloads=None, as_array: bool = False):
    """Write the tensors and their encoded planes as a compact container
    (\\x89PTWC) or, for one tensor, a compact frame (\\x89PTWS) through
    ptwm_mi355x_container_write.  With ``payloads`` (host bytes or a numpy
    uint8 array) every plane's payload is an (offset, length) span of it,
    and nothing is copied on the way in; ``as_array`` returns the file as a
    numpy uint8 array instead of bytes."""
    import struct

    import numpy as np

    if layout not in ("compact", "frame"):
        raise ValueError(f"container_write: unknown layout {layout!r}")
    spec = bytearray(struct.pack("<IHHI", 0x57575450, 1, 1 if layout == "compact" else 2, len(tensors)))
    blob = bytearray()
    for t in tensors:
        nm = t.name.encode()
        spec += struct.pack("<H", len(nm)) + nm
        spec += struct.pack("<HBBB", t.dtype_code, t.input_format, t.chain, len(t.shape))
        spec += b"".join(struct.pack("<Q", d) for d in t.shape)
        spec += struct.pack("<B", 1 if t.xxh64 is not None else 0)
        if t.xxh64 is not None:
            spec += struct.pack("<Q", t.xxh64)
        spec += struct.pack("<B", len(t.planes))
        for p in t.planes:
            fl = (1 if p.crc32 is not None else 0) | (2 if p.chunks is not None else 0)
            spec += struct.pack("<HB", p.codec, fl)
            if p.crc32 is not None:
                spec += struct.pack("<I", p.crc32)
            if isinstance(p.payload, tuple) != (payloads is not None):
                raise ValueError("container_write: give every payload as a span of `payloads`, or none")
            if payloads is not None:
                spec += struct.pack("<QQ", *p.payload)
            else:
                spec += struct.pack("<QQ", len(blob), len(p.payload))
                blob += p.payload
            if p.chunks is not None:
                spec += struct.pack("<I", len(p.chunks)) + b"".join(struct.pack("<II", a, b) for a, b in p.chunks)
    L = lib()
    spec = bytes(spec)
    bptr, blen, keep = _host_buf(payloads if payloads is not None else bytes(blob))
    n = C.c_size_t(0)
    cap = blen + 2 * len(spec) + 65536  # enough for the file: payloads plus overheads of the spec's size
    while True:
        out = np.empty(cap, np.uint8)
        rc = L.ptwm_mi355x_container_write(spec, len(spec), bptr, blen, C.c_void_p(int(out.ctypes.data)), cap,
                                           C.byref(n))
        if rc == RC_BUFFER_TOO_SMALL and n.value > cap:
            cap = n.value
            continue
        break
    check(rc, "container_write")
    del keep
    return out[:n.value] if as_array else out[:n.value].tobytes()
