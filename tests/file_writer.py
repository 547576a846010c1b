"""GPU encoder plans -> container writer input (test helper, not a test).

A PTMD plan from one of the library's GPU encoders names, per plane, the
codec, the payload's span in the encoder's output buffer, the chunk table
(offset_in_payload, decoded_size) as plane_record.rs:16-20 stores it, the
plane CRC-32 and the tensor XXH64.  ``write_tensors`` turns such plans into
``api.WriteTensor``s whose payloads are spans of the host copy of that
buffer, so a whole model is written without copying each payload.
"""
from __future__ import annotations

from ptwm_amd import api


def write_tensors(entries, base: int = 0):
    """``entries``: (name, public dtype code, shape, TensorPlan) whose payload
    offsets are relative to ``base`` in the payload buffer."""
    out = []
    for name, dtype_code, shape, t in entries:
        planes = [api.WritePlane(p.codec, (base + p.payload_offset, p.payload_len), p.crc32,
                                 [tuple(c) for c in p.chunks] if p.chunks is not None else None)
                  for p in t.planes]
        out.append(api.WriteTensor(name, dtype_code, t.chain, shape, planes, t.xxh64))
    return out
