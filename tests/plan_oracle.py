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


def _o1sac_plane(data: bytes, p: P.PlanePlan, payload: bytes) -> bytes:
    """Order1ScaleAC: the plane's state (or each chunk frame's own, container.rs:2010-2049)."""
    off, ln, row_len, ver = p.state
    if p.chunks is None:
        return O.o1sac_decode(bytes(data[off:off + ln]), payload, p.plane_len, row_len, ver)
    out = b""
    for k, (start, size) in enumerate(p.chunks):
        end = p.chunks[k + 1][0] if k + 1 < len(p.chunks) else len(payload)
        frame = payload[start:end]
        sl = int.from_bytes(frame[1:5], "little")
        out += O.o1sac_decode(frame[5:5 + sl], frame[5 + sl:], size, row_len, frame[0])
    return out


def decode_tensor(data: bytes, t: P.TensorPlan) -> bytes:
    planes = []
    for p in t.planes:
        payload = bytes(data[p.payload_offset:p.payload_offset + p.payload_len])  # data: bytes or a uint8 array
        if p.codec == O.CODEC_O1SAC:
            plane = _o1sac_plane(data, p, payload)
        elif p.chunks is not None:
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
