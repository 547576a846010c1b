"""The library's container writers on the CPU (no GPU).

- Round trips: every compact container (\\x89PTWC), compact frame
  (\\x89PTWS) and legacy container (\\x89PTWM) the reference wrote
  (tests/golden: the fuzz corpus files, the legacy files of its
  compatibility tests and the 28 frames of its compact-frame tests) is read
  into its sections and records and written again through the writer
  (ptwc.rs, extension/compact_table.rs, tensor_record_compact.rs,
  chain/wire_compact.rs, compact.rs; container.rs:790-1060, header.rs,
  tensor_record.rs, plane_record.rs, chain/wire.rs, index.rs), and comes
  back byte for byte.  The legacy header's Extension Table hash is BLAKE3
  recomputed by the writer; the reader refuses a table that does not match
  it (container.rs:1299).  The writer recomputes the
  header lengths and meta_xxh64, the registry, the index and the footer,
  and re-decides the implicit spine edges, bound Sources and the frame's
  stored orig_size, so a wrong rule shows as a byte difference.
- The writer is not a copier: a record whose payload is changed, or a
  tensor dropped from the model, changes the bytes in the places the
  format fixes (tested through new files below).
- New files: tensors of every decode-plan chain, planes encoded by the
  oracle in the reference formats (Huffman, rANS, Identity, chunked) and in
  this library's huff_ilv / rans_ilv, written as a compact container and as
  frames, then opened by the library's reader (ptwm_mi355x_container_plan)
  and decoded by the oracle to the original bytes, with the plane CRC-32s
  and XXH64s the files carry checked; a written file also round-trips
  through the rewriter.
"""
import glob
import os

import numpy as np
import pytest

import oracle as O
from ptwm_amd import api, ids, plan as P

import plan_oracle

HERE = os.path.dirname(os.path.abspath(__file__))
COMPACT = sorted(glob.glob(os.path.join(HERE, "golden", "ptwm_files", "ptwc_*")))
LEGACY = sorted(glob.glob(os.path.join(HERE, "golden", "ptwm_files", "legacy_*")))
FRAMES = sorted(glob.glob(os.path.join(HERE, "golden", "ptws_frames", "*.body")))

# public dtype codes (dtype.rs:79-103)
DT_F32, DT_BF16, DT_U8, DT_E4M3, DT_E5M2 = 1, 6, 13, 29, 30


@pytest.mark.parametrize("path", COMPACT, ids=[os.path.basename(p) for p in COMPACT])
def test_compact_container_round_trip(path):
    data = open(path, "rb").read()
    assert api.container_rewrite(data) == data


@pytest.mark.parametrize("path", FRAMES, ids=[os.path.basename(p) for p in FRAMES])
def test_frame_round_trip(path):
    data = b"\x89PTWS" + open(path, "rb").read()
    assert api.container_rewrite(data) == data


@pytest.mark.parametrize("path", LEGACY, ids=[os.path.basename(p) for p in LEGACY])
def test_legacy_container_round_trip(path):
    data = open(path, "rb").read()
    assert api.container_rewrite(data) == data


def test_legacy_header_hash_is_blake3_of_the_table():
    assert LEGACY
    for path in LEGACY:
        data = open(path, "rb").read()
        et_off, et_len = (int.from_bytes(data[k:k + 8], "little") for k in (11, 19))
        assert et_off == 91 and et_len > 0
        assert data[27:59] == O.blake3(data[et_off:et_off + et_len]), path


def test_legacy_reader_refuses_a_table_that_misses_its_hash():
    data = open(LEGACY[0], "rb").read()
    api.container_plan(data)
    for at in (91 + 4, 91 + 40):  # a byte of the table's first entry (canonical id, label)
        bad = bytearray(data)
        bad[at] ^= 0xFF
        with pytest.raises(Exception):
            api.container_plan(bytes(bad))
    bad = bytearray(data)
    bad[30] ^= 1  # the stored hash itself
    with pytest.raises(Exception):
        api.container_plan(bytes(bad))


def test_rewrite_rejects_a_broken_file():
    data = bytearray(open(COMPACT[0], "rb").read())
    data[12] ^= 0x40  # an Extension Table length no longer matching its section
    with pytest.raises(Exception):
        api.container_rewrite(bytes(data))


def tensors(seed: int):
    """One tensor per decode-plan chain, with its bytes."""
    rng = np.random.default_rng(seed)
    g = rng.standard_normal
    bf16 = (g(3 * 1024 + 16).astype(np.float32) * 0.02).view(np.uint32)
    bf16 = ((bf16 + 0x7FFF + ((bf16 >> 16) & 1)) >> 16).astype(np.uint16)  # round to bfloat16
    out = [
        ("w.bf16", DT_BF16, P.CHAIN_IEEE16_SPLIT2, [len(bf16)], bf16.tobytes()),
        ("w.fp32", DT_F32, P.CHAIN_IEEE32_SPLIT4, [40, 50], (g(2000) * 0.02).astype(np.float32).tobytes()),
        ("w.fp8", DT_E4M3, P.CHAIN_E4M3_NIBBLE, [64, 40], rng.integers(0, 126, 2560, np.uint8).tobytes()),
        ("w.e5m2", DT_E5M2, P.CHAIN_E5M2_NIBBLE, [700], rng.integers(0, 122, 700, np.uint8).tobytes()),
        ("w.mxfp4", DT_U8, P.CHAIN_NIBBLE_SPLIT, [32, 64], rng.integers(0, 256, 2048, np.uint8).tobytes()),
        ("w.scales", DT_U8, P.CHAIN_PASSTHROUGH, [32, 2],
         np.clip(np.round(g(64) * 1.5 - 6) + 127, 0, 255).astype(np.uint8).tobytes()),
    ]
    return out


def encode_plane(codec: str, plane: bytes):
    """(wire id, payload, chunks) for a codec choice."""
    if codec == "huffman":
        return O.CODEC_HUFFMAN, O.codec_encode(O.CODEC_HUFFMAN, plane), None
    if codec == "rans":
        return O.CODEC_RANS, O.codec_encode(O.CODEC_RANS, plane), None
    if codec == "identity":
        return O.CODEC_IDENTITY, O.codec_encode(O.CODEC_IDENTITY, plane), None
    if codec == "chunked":
        pay, ent = O.encode_plane_chunked(O.CODEC_HUFFMAN, plane, 512)
        return O.CODEC_HUFFMAN, pay, [tuple(int(v) for v in e) for e in ent]
    if codec == "huff_ilv":
        return ids.CODEC_HUFF_ILV, O.ilv_encode(plane), None
    if codec == "rans_ilv":
        return ids.CODEC_RANS_ILV, O.rans_ilv_encode(plane), None
    raise ValueError(codec)


CODEC_CYCLE = ["huffman", "rans", "identity", "chunked", "huff_ilv", "rans_ilv"]


def write_model(seed: int, crc: bool, hsh: bool, layout: str = "compact", codecs=CODEC_CYCLE):
    items, raws = [], []
    for k, (name, dt, chain, shape, raw) in enumerate(tensors(seed)):
        planes = []
        for j, plane in enumerate(O.chain_forward(chain, raw)):
            codec, pay, ch = encode_plane(codecs[(k + j) % len(codecs)], plane)
            planes.append(api.WritePlane(codec, pay, O.crc32(plane) if crc else None, ch))
        items.append(api.WriteTensor(name, dt, chain, shape, planes, O.xxh64(raw) if hsh else None))
        raws.append((name, raw))
    return items, raws


def open_and_decode(data: bytes, raws, named: bool = True):
    plan, ents, out_len = api.container_plan(data)
    assert [e.name for e in ents] == ([n for n, _ in raws] if named else [""])   # a frame has no name
    assert all(e.status == 0 and e.plan_index >= 0 for e in ents)
    got = plan_oracle.decode_plan(data, plan, out_len)
    for e, (_, raw) in zip(ents, raws):
        assert got[e.out_offset:e.out_offset + e.orig_size] == raw, e.name
    return ents


@pytest.mark.parametrize("crc,hsh", [(False, False), (True, False), (False, True), (True, True)])
def test_written_compact_container_opens_and_decodes(crc, hsh):
    items, raws = write_model(3, crc, hsh)
    data = api.container_write(items)
    assert data[:9] == b"\x89PTWC\r\n\x1a\n" and data[-8:] == b"\x89TWMEOF\x1a"
    ents = open_and_decode(data, raws)
    assert all(e.crc_checked == crc and e.hash_checked == hsh for e in ents)
    assert api.container_rewrite(data) == data


def test_written_file_depends_on_every_payload_byte_and_tensor():
    items, raws = write_model(5, True, True)
    a = api.container_write(items)
    items[2].planes[0].payload = bytes([items[2].planes[0].payload[0] ^ 1]) + items[2].planes[0].payload[1:]
    b = api.container_write(items)
    assert len(a) == len(b) and sum(x != y for x, y in zip(a, b)) == 1  # only that payload byte
    c = api.container_write(items[:2] + items[3:])
    plan, ents, _ = api.container_plan(c)
    assert [e.name for e in ents] == [n for k, (n, _) in enumerate(raws) if k != 2]


def test_written_frames_open_and_decode():
    items, raws = write_model(7, True, False, codecs=["huffman", "rans", "identity"])
    for it, raw in zip(items, raws):
        data = api.container_write([it], layout="frame")
        assert data[:5] == b"\x89PTWS"
        open_and_decode(data, [raw], named=False)
        assert api.container_rewrite(data) == data
    it = items[0]
    it.xxh64 = O.xxh64(raws[0][1])  # hash and plane CRCs: the frame keeps the hash only
    data = api.container_write([it], layout="frame")
    ents = open_and_decode(data, [raws[0]], named=False)
    assert ents[0].hash_checked and not ents[0].crc_checked


def test_write_refuses_what_the_layout_cannot_hold():
    items, _ = write_model(9, False, False)
    with pytest.raises(Exception) as ei:
        api.container_write(items[3:4], layout="frame")  # chunks and huff_ilv in a frame
    assert getattr(ei.value, "rc", None) in (-1, -5)
    bad = api.WriteTensor("x", DT_BF16, P.CHAIN_IEEE32_SPLIT4, [8], [])
    with pytest.raises(Exception):
        api.container_write([bad])                       # a dtype the chain cannot take
    dup = write_model(9, False, False)[0]
    with pytest.raises(Exception):
        api.container_write([dup[0], dup[0]])            # duplicate names


def test_payload_spans_of_one_buffer_write_the_same_file():
    """Payloads handed over as spans of one host buffer (how a GPU-encoded
    model comes back from the device) write the same file, also as an array."""
    items, raws = write_model(11, True, True)
    want = api.container_write(items)
    buf, spans = bytearray(b"\xee" * 13), []
    for t in items:
        for p in t.planes:
            spans.append((len(buf), len(p.payload)))
            buf += p.payload + b"\xee" * 7  # gaps the spans skip
    k = 0
    for t in items:
        for i, p in enumerate(t.planes):
            t.planes[i] = api.WritePlane(p.codec, spans[k], p.crc32, p.chunks)
            k += 1
    arr = np.frombuffer(bytes(buf), np.uint8)
    got = api.container_write(items, payloads=arr, as_array=True)
    assert isinstance(got, np.ndarray) and got.tobytes() == want
    assert api.container_write(items, payloads=bytes(buf)) == want
    open_and_decode(got.tobytes(), raws)
    plan, ents, out_len = api.container_plan(got)  # the reader takes the array as it is
    plan2, ents2, out_len2 = api.container_plan(want)
    assert (plan, out_len) == (plan2, out_len2)
    assert [e.name for e in ents] == [e.name for e in ents2] == [n for n, _ in raws]
    with pytest.raises(ValueError):
        api.container_write(items)  # spans without the buffer


def _leb(v: int) -> bytes:
    out = bytearray()
    while v >= 0x80:
        out.append((v & 0x7F) | 0x80)
        v >>= 7
    out.append(v)
    return bytes(out)


def o1sac_frame(rows: int, row_len: int, seed: int = 4):
    """A compact frame holding an E8M0-like scale tensor [rows, row_len] as
    one Order1ScaleAC plane with its state inline (compact.rs:479-505: head
    (codec << 2 | 1), version, state, payload).  Written through the
    library's frame writer with an Identity plane, whose tail is then
    replaced.  Returns (frame, plane, state)."""
    from test_oracle_o1sac import make_state

    rng = np.random.default_rng(seed)
    plane = np.clip(np.round(rng.normal(-6, 1.5, rows * row_len)) + 127, 0, 255).astype(np.uint8).tobytes()
    st = make_state(rng, sorted(set(plane)), skew=2.0)
    ident = O.codec_encode(O.CODEC_IDENTITY, plane)
    base = api.container_write([api.WriteTensor("s", DT_U8, P.CHAIN_PASSTHROUGH, [rows, row_len],
                                                [api.WritePlane(O.CODEC_IDENTITY, ident)])], layout="frame")
    tail = b"\x00" + _leb(len(ident)) + ident          # head 0 (Identity, no state), length, payload
    assert base.endswith(tail)
    pay = O.o1sac_encode(st, plane, row_len)
    frame = base[:-len(tail)] + _leb((O.CODEC_O1SAC << 2) | 1) + b"\x01" + _leb(len(st)) + st + _leb(len(pay)) + pay
    return frame, plane, st


@pytest.mark.parametrize("rows,row_len", [(64, 128), (7, 33), (1, 500)])
def test_frame_order1scaleac_plane_plans_with_its_state_and_rows(rows, row_len):
    """A frame's Order1ScaleAC plane decodes with its inline state and the
    rows of the Source's last dimension (transforms/source.rs:145-176), as
    the reference's decode_body passes legacy_plane_layout(descriptor.layout)
    to the codec (compact.rs:479-505)."""
    frame, plane, st = o1sac_frame(rows, row_len)
    plan, ents, out_len = api.container_plan(frame)
    assert ents[0].status == 0 and ents[0].plan_index == 0
    t = P.decode_plan(plan)[0]
    assert [p.codec for p in t.planes] == [O.CODEC_O1SAC]
    off, ln, rl, ver = t.planes[0].state
    assert (frame[off:off + ln], rl, ver) == (st, row_len, 1)
    assert plan_oracle.decode_plan(frame, plan, out_len)[:len(plane)] == plane
    # a flat layout would code the plane as one row: the row length matters
    if rows > 1:
        assert O.o1sac_encode(st, plane, 0) != O.o1sac_encode(st, plane, row_len)
