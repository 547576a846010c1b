"""Config 5 at full size as files: MXFP4 weights 14336x2048 (two FP4 codes
per byte, nibble split) and their E8M0 scales 14336x128 (one byte plane),
encoded on the GPU, written by the library's container writer, read back by
its reader and restored on the GPU.

- Reference formats (the reference's encoder output
  "round-trip through the container"): every plane payload the GPU encoder
  writes equals the oracle's restatement of the reference encoder on the
  full tensor (O.codec_encode for whole payloads, O.encode_plane_chunked
  for the 256 KiB chunk frames of python/ptwm/_config.py:151), for Huffman
  and rANS; the compact container (\\x89PTWC) and one compact frame
  (\\x89PTWS) per tensor written from those payloads, with plane CRC-32s
  and tensor XXH64s, re-open in ptwm_mi355x_container_plan, restore
  bit-exact on the GPU with both checked, and decode to the same bytes in
  the oracle.
- GPU-native formats: the two tensors encoded with huff_ilv / rans_ilv in
  one batched call, written as a compact container (the codecs' 0x7F
  Extension Table entries), re-opened, restored in one call (the two-chain
  launch) and decoded by the oracle's restatement of the formats.
"""
import sys

import numpy as np
import pytest

import bench
import oracle as O
from ptwm_amd import api, ids, plan as P

import file_writer
import plan_oracle

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

DT_U8 = 13  # dtype.rs:79-103: the packed FP4 pairs and the E8M0 scales are stored as bytes
SPECS = [("mlp.experts.0.down_proj.weight_packed", (14336, 2048), "fp4", P.CHAIN_NIBBLE_SPLIT),
         ("mlp.experts.0.down_proj.weight_scale", (14336, 128), "e8m0", P.CHAIN_PASSTHROUGH)]
HUF, RANS = O.CODEC_HUFFMAN, O.CODEC_RANS


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def host(t) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def to_device(a: np.ndarray):
    t = torch.empty(max(1, a.size), dtype=torch.uint8, device="cuda:0")
    if a.size:
        a = np.ascontiguousarray(a)
        t[: a.size].copy_(torch.from_numpy(a if a.flags.writeable else a.copy()))
    return t[: a.size]


def restore(plan_bytes: bytes, src, out_len: int):
    out = torch.full((out_len,), 0xA5, dtype=torch.uint8, device="cuda:0")
    n = api.hardware_backend_dispatch_decode_cuda(ids.HARDWARE_BACKEND_LABEL, ids.DECODE_PLAN_LABEL, plan_bytes,
                                                  src, out, 0)
    torch.cuda.synchronize()
    return n, out


@pytest.fixture(scope="module")
def c5():
    items = []
    for i, (name, shape, kind, chain) in enumerate(SPECS):
        raw = bench.gen_tensor(kind, shape, 500 + i)
        items.append((name, shape, chain, raw, host(raw).tobytes()))
    note(f"config 5: {[(n, s) for n, s, *_ in items]} generated")
    yield items


def check_file(data, items, crc: bool, hsh: bool, named: bool = True):
    """Re-open a written file, restore it on the GPU and in the oracle."""
    plan_bytes, ents, out_len = api.container_plan(data)
    assert [e.name for e in ents] == ([n for n, *_ in items] if named else [""])  # a frame has no name
    assert all(e.status == 0 and e.plan_index >= 0 for e in ents)
    assert all(e.crc_checked == crc and e.hash_checked == hsh for e in ents)
    src = to_device(np.frombuffer(data, np.uint8) if isinstance(data, bytes) else data)
    n, out = restore(plan_bytes, src, out_len)
    assert n == sum(len(it[4]) for it in items)
    for e, (name, _, _, raw, _) in zip(ents, items):
        assert torch.equal(out[e.out_offset:e.out_offset + e.orig_size], raw), name
    want = plan_oracle.decode_plan(bytes(data), plan_bytes, out_len)
    for e, (name, _, _, _, hb) in zip(ents, items):
        assert want[e.out_offset:e.out_offset + e.orig_size] == hb, name
    return ents


@pytest.mark.parametrize("codec,chunk", [(HUF, 0), (RANS, 0), (HUF, bench.REF_CHUNK)],
                         ids=["huffman", "rans", "huffman-chunked"])
def test_config5_reference_format_bytes_and_files(c5, codec, chunk):
    cap = sum(len(it[4]) for it in c5) + 65536 * len(c5) + (1 << 20)
    blob = torch.empty(cap, dtype=torch.uint8, device="cuda:0")
    off, entries = 0, []
    for name, shape, chain, raw, hb in c5:
        used, st = api.encode_tensor_ref_cuda(chain, [codec] * P.CHAIN_PLANES[chain], chunk, raw, blob[off:], 0)
        t = P.decode_plan(st)[0]
        for p in t.planes:
            p.payload_offset += off
        for p, c in zip(t.planes, api.plane_crc32_cuda(chain, raw, 0)):
            p.crc32 = c
        t.xxh64 = api.xxh64_cuda(raw, 0)
        entries.append((name, DT_U8, list(shape), t))
        off = (off + used + 255) // 256 * 256
    payloads = host(blob[:off])
    # the GPU encoder's bytes are the reference encoder's, on the full tensors
    for (name, _, chain, _, hb), (_, _, _, t) in zip(c5, entries):
        planes = O.chain_forward(chain, hb)
        for p, plane in zip(t.planes, planes):
            got = payloads[p.payload_offset:p.payload_offset + p.payload_len].tobytes()
            assert p.codec == codec and p.crc32 == O.crc32(plane), name
            if chunk:
                pay, ent = O.encode_plane_chunked(codec, plane, chunk)
                assert got == pay and [tuple(c) for c in p.chunks] == [tuple(int(v) for v in e) for e in ent], name
            else:
                assert got == O.codec_encode(codec, plane), name
        assert t.xxh64 == O.xxh64(hb), name
    note(f"config 5 {codec}/{chunk}: GPU payloads == oracle encode ({off} bytes)")
    data = api.container_write(file_writer.write_tensors(entries), payloads=payloads, as_array=True)
    note(f"config 5 {codec}/{chunk}: compact container {data.size} bytes")
    assert data[:9].tobytes() == b"\x89PTWC\r\n\x1a\n"
    check_file(data, c5, True, True)
    assert api.container_rewrite(data.tobytes()) == data.tobytes()
    if not chunk:  # a frame holds whole payloads; with the XXH64 it drops the plane CRCs (compact.rs)
        for ent, item in zip(entries, c5):
            frame = api.container_write(file_writer.write_tensors([ent]), layout="frame", payloads=payloads)
            assert frame[:5] == b"\x89PTWS"
            check_file(frame, [item], False, True, named=False)
        note(f"config 5 {codec}: frames restored")


@pytest.mark.parametrize("codec", ["huff_ilv", "rans_ilv"])
def test_config5_native_format_file(c5, codec):
    cap = sum(len(it[4]) for it in c5) + 65536 * len(c5) + (1 << 20)
    blob = torch.empty(cap, dtype=torch.uint8, device="cuda:0")
    used, st = api.encode_tensors_cuda([(chain, raw) for _, _, chain, raw, _ in c5], blob, 0, codec=codec)
    plans = P.decode_plan(st)
    assert {p.codec for t in plans for p in t.planes} <= {0, ids.CODEC_HUFF_ILV, ids.CODEC_RANS_ILV}
    for (_, _, chain, raw, _), t in zip(c5, plans):
        for p, c in zip(t.planes, api.plane_crc32_cuda(chain, raw, 0)):
            p.crc32 = c
        t.xxh64 = api.xxh64_cuda(raw, 0)
    payloads = host(blob[:used])
    entries = [(name, DT_U8, list(shape), t) for (name, shape, *_), t in zip(c5, plans)]
    data = api.container_write(file_writer.write_tensors(entries), payloads=payloads, as_array=True)
    note(f"config 5 {codec}: compact container {data.size} bytes, planes "
         f"{[hex(p.codec) for t in plans for p in t.planes]}")
    check_file(data, c5, True, True)
