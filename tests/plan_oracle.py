"""CPU decode of a PTMD plan with the oracle (test helper, not a test).

Each planned tensor's planes are decoded from the input bytes with the
oracle's codec restatements (whole payloads or chunk frames), checked
against the plan's CRC-32s, passed through the inverse of their plane op,
merged by the oracle's chain inverse and checked
against the plan's XXH64 -- what container.rs:1795-2196 does per tensor.
"""
from __future__ import annotations

import oracle as O
from ptwm_amd import plan as P

HUFF_ILV, RANS_ILV = 0x7F01, 0x7F02  # this library's GPU-native codecs (their specification is the oracle's)


def decode_tensor(data: bytes, t: P.TensorPlan) -> bytes:
    planes = []
    for p in t.planes:
        payload = data[p.payload_offset:p.payload_offset + p.payload_len]
        if p.chunks is not None:
            plane = O.decode_plane_chunked(p.codec, payload, p.chunks)
        elif p.codec == HUFF_ILV:
            plane = O.ilv_decode(payload, p.plane_len)
        elif p.codec == RANS_ILV:
            plane = O.rans_ilv_decode(payload, p.plane_len)
        else:
            plane = O.codec_decode(p.codec, payload, p.plane_len)
        assert len(plane) == p.plane_len
        if p.crc32 is not None:
            assert O.crc32(plane) == p.crc32
        planes.append(O.plane_op(p.op, p.op_param, plane, inverse=True))
    raw = O.chain_inverse(t.chain, planes)
    assert len(raw) == t.out_len
    if t.xxh64 is not None:
        assert O.xxh64(raw) == t.xxh64
    return raw


def decode_plan(data: bytes, plan_bytes: bytes, out_len: int) -> bytes:
    out = bytearray(out_len)
    for t in P.decode_plan(plan_bytes):
        out[t.out_offset:t.out_offset + t.out_len] = decode_tensor(data, t)
    return bytes(out)
