"""Decode plans: the state bytes of the tensor-level entry point.

A plan lists tensors the way the container stores them
(crates/ptwm-core/src/container.rs:1795-2196): per tensor its chain and, per
plane, the codec wire id, the payload's offset and length in the input
buffer, the decoded plane length, an optional CRC32 and the chunk table
(plane_record.rs:16-20: ``(offset_in_payload u32, decoded_size u32)``), and
per tensor an optional payload hash (container.rs:2185-2194: xxh64, seed 0,
of the restored bytes).
Binary layout (little endian), "PTMD" version 1:

    u32 magic 0x444D5450 | u16 version=1 | u16 flags=0 | u32 n_tensors
    tensor: u64 out_offset | u64 out_len | u8 chain | u8 n_planes | u16 flags (bit0 crc, bit1 hash)
            | [u64 xxh64 (seed 0) of the restored tensor if hash flag]
      plane: u16 codec | u16 flags | u32 n_chunks
             | u64 payload_offset | u64 payload_len | u64 plane_len
             | [u32 crc32 if tensor crc flag]
             | [u64 state_offset | u32 state_len | u32 row_len | u32 state_version if plane flag bit 6]
             | n_chunks x (u32 offset, u32 size)
      plane flags: bit0 chunked; bits 1-2 the inverse plane op applied to the
      decoded plane before the merge (0 none, 1 IntDelta, 2 PredictorXor,
      3 MantissaZeroStrip: chain/dispatch.rs:96-122); bits 3-5 its parameter
      (log2 of the element width for IntDelta / PredictorXor, k for the strip).
      The plane CRC covers the decoded plane, before the op (container.rs:2152-2170).
      Bit 6: the codec state and plane layout of an Order1ScaleAC plane
      (codecs/order1_scale_ac.rs): the state bytes in the input buffer (a
      chunked plane's chunk frames carry their own), their format version and
      the row length (0 = Flat); required for that codec, refused for others.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

CHAIN_IEEE16_SPLIT2 = 1
CHAIN_IEEE32_SPLIT4 = 2
CHAIN_E4M3_NIBBLE = 3
CHAIN_E5M2_NIBBLE = 4
CHAIN_NIBBLE_SPLIT = 5
CHAIN_PASSTHROUGH = 6
CHAIN_PLANES = {1: 2, 2: 4, 3: 2, 4: 2, 5: 2, 6: 1}
CHAIN_RATIO = {1: 2, 2: 4, 3: 1, 4: 1, 5: 1, 6: 1}
MAGIC = 0x444D5450
PLANE_OP_NONE = 0
PLANE_OP_INT_DELTA = 1
PLANE_OP_PREDICTOR_XOR = 2
PLANE_OP_MANTISSA_ZERO_STRIP = 3


@dataclass
class PlanePlan:
    codec: int
    payload_offset: int
    payload_len: int
    plane_len: int
    chunks: list[tuple[int, int]] | None = None   # (offset_in_payload, decoded_size)
    crc32: int | None = None
    op: int = PLANE_OP_NONE   # inverse plane op after the decode
    op_param: int = 0         # element width in bytes (deltas) or k (strip)
    state: tuple[int, int, int, int] | None = None  # (offset, length, row_len, version): Order1ScaleAC


@dataclass
class TensorPlan:
    chain: int
    out_offset: int
    out_len: int
    planes: list[PlanePlan] = field(default_factory=list)
    xxh64: int | None = None


def _plane_flags(p: PlanePlane) -> int:
    f = (1 if p.chunks is not None else 0) | (0x40 if p.state is not None else 0)
    if p.op == PLANE_OP_NONE:
        return f
    code = p.op_param if p.op == PLANE_OP_MANTISSA_ZERO_STRIP else p.op_param.bit_length() - 1
    return f | (p.op << 1) | (code << 3)


def encode_plan(tensors: list[TensorPlan]) -> bytes:
    out = bytearray(struct.pack("<IHHI", MAGIC, 1, 0, len(tensors)))
    for t in tensors:
        has_crc = any(p.crc32 is not None for p in t.planes)
        tflags = (1 if has_crc else 0) | (2 if t.xxh64 is not None else 0)
        out += struct.pack("<QQBBH", t.out_offset, t.out_len, t.chain, len(t.planes), tflags)
        if t.xxh64 is not None:
            out += struct.pack("<Q", t.xxh64)
        for p in t.planes:
            ch = p.chunks or []
            out += struct.pack("<HHIQQQ", p.codec, _plane_flags(p), len(ch),
                               p.payload_offset, p.payload_len, p.plane_len)
            if has_crc:
                out += struct.pack("<I", p.crc32 or 0)
            if p.state is not None:
                out += struct.pack("<QIII", *p.state)
            for off, size in ch:
                out += struct.pack("<II", off, size)
    return bytes(out)


def decode_plan(buf: bytes) -> list[TensorPlan]:
    magic, ver, flags, n = struct.unpack_from("<IHHI", buf, 0)
    if magic != MAGIC or ver != 1 or flags != 0:
        raise ValueError("not a PTMD v1 plan")
    o = 12
    res = []
    for _ in range(n):
        off, ln, chain, np_, tfl = struct.unpack_from("<QQBBH", buf, o)
        o += 20
        t = TensorPlan(chain, off, ln)
        if tfl & 2:
            (t.xxh64,) = struct.unpack_from("<Q", buf, o)
            o += 8
        for _ in range(np_):
            codec, pfl, nch, po, pl, plen = struct.unpack_from("<HHIQQQ", buf, o)
            o += 32
            crc = None
            if tfl & 1:
                (crc,) = struct.unpack_from("<I", buf, o)
                o += 4
            state = None
            if pfl & 0x40:
                state = struct.unpack_from("<QIII", buf, o)
                o += 20
            chunks = None
            if pfl & 1:
                chunks = [struct.unpack_from("<II", buf, o + 8 * k) for k in range(nch)]
                o += 8 * nch
            op, code = (pfl >> 1) & 3, (pfl >> 3) & 7
            param = 0 if op == PLANE_OP_NONE else code if op == PLANE_OP_MANTISSA_ZERO_STRIP else 1 << code
            t.planes.append(PlanePlan(codec, po, pl, plen, chunks, crc, op, param, state))
        res.append(t)
    if o != len(buf):
        raise ValueError("trailing bytes in plan")
    return res
