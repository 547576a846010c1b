"""Container reader (ptwm_mi355x_container_plan) on CPU.

The reference's own files are the fixtures: its golden legacy containers
(crates/ptwm-core/tests/fixtures/legacy_*.ptwm, EXPECTED (len, xxh64) in
legacy_fixtures.rs:63-123 = tests/golden/legacy_xxh64.json), its PTWC
corpus (fuzz/corpus/container_open/ptwc_*) and its PTWS frames
(fuzz/corpus/compact_decode/*, stored without the magic as the fuzz target
does).  The reader is host code; the decode here is the oracle's, so these
tests pin the reader's plans and, through the fixtures' CRCs and hashes,
the oracle's codecs.
"""
import glob
import json
import os

import numpy as np
import pytest

import oracle as O
from ptwm_amd import api, plan as P
from ptwm_amd._native import NativeError

import plan_oracle

HERE = os.path.dirname(os.path.abspath(__file__))
FILES = os.path.join(HERE, "golden", "ptwm_files")
FRAMES = os.path.join(HERE, "golden", "ptws_frames")
EXPECTED = json.load(open(os.path.join(HERE, "golden", "legacy_xxh64.json")))
PTWS = b"\x89PTWS"


def _read(path):
    with open(path, "rb") as f:
        return f.read()


def _legacy():
    return sorted(glob.glob(os.path.join(FILES, "legacy_*.ptwm")))


def _frames():
    return sorted(glob.glob(os.path.join(FRAMES, "*.body")))


@pytest.mark.parametrize("path", _legacy(), ids=os.path.basename)
def test_legacy_tensors_listed_in_record_order(path):
    _, ents, _ = api.container_plan(_read(path))
    names = [e.name for e in ents]
    if "p4_byte_fp32" in path:
        assert [(e.name, e.orig_size) for e in ents] == [("p4.byte.fp32", 512)]
        return
    order = [n for n in EXPECTED if n in names]
    assert names == order  # legacy_fixtures.rs writes them in this order
    for e in ents:
        assert e.orig_size == EXPECTED[e.name][0]


@pytest.mark.parametrize("path", _legacy() + sorted(glob.glob(os.path.join(FILES, "ptwc_*"))),
                         ids=os.path.basename)
def test_planned_tensors_decode_to_the_expected_hashes(orc, path):
    data = _read(path)
    plan, ents, out_len = api.container_plan(data)
    out = plan_oracle.decode_plan(data, plan, out_len)  # checks every CRC and hash the plan carries
    tensors = P.decode_plan(plan)
    assert len(tensors) == sum(e.plan_index >= 0 for e in ents)
    for e in ents:
        if e.plan_index < 0:
            # not decoded on the device: Zstd / Order1ScaleAC planes (-5)
            assert e.status == -5
            continue
        t = tensors[e.plan_index]
        assert (t.out_offset, t.out_len, t.chain) == (e.out_offset, e.orig_size, e.chain)
        assert e.out_offset % 256 == 0
        raw = out[e.out_offset:e.out_offset + e.orig_size]
        if e.name in EXPECTED:
            assert "%016x" % orc.xxh64(raw) == EXPECTED[e.name][1]
        assert e.hash_checked and t.xxh64 == orc.xxh64(raw)


def test_chunked_tans_tensor_is_planned_with_its_chunk_tables():
    _, ents, _ = api.container_plan(_read(os.path.join(FILES, "legacy_v1_1_0.ptwm")))
    e = [x for x in ents if x.name == "model.layers.2.chunked.weight"][0]
    assert e.status == 0 and e.chain == 1 and e.crc_checked and e.hash_checked
    plan, _, _ = api.container_plan(_read(os.path.join(FILES, "legacy_v1_1_0.ptwm")))
    t = P.decode_plan(plan)[e.plan_index]
    assert [p.codec for p in t.planes] == [0x0000, 0x0007]
    assert t.planes[0].chunks == [(0, 256), (261, 256)]
    assert t.planes[1].chunks == [(0, 256), (132, 256)]


@pytest.mark.parametrize("path", _frames(), ids=os.path.basename)
def test_ptws_frames(orc, path):
    body = _read(path)
    frame = PTWS + body
    plan, ents, out_len = api.container_plan(frame)
    assert len(ents) == 1
    e = ents[0]
    assert e.name == "" and e.hash_checked == path.endswith("_hash.body")
    if e.plan_index >= 0:
        out = plan_oracle.decode_plan(frame, plan, out_len)  # checks the frame's hash / CRCs
        raw = out[:e.orig_size]
        if body[0] & 0x20:  # FLAG_STORED: the body is the raw bytes
            assert raw == frame[len(frame) - e.orig_size:]
    else:
        assert e.status == -5


@pytest.mark.parametrize("name,plane", [("bf16_smooth", 1), ("fp32_smooth", 3), ("byte_bf16", 1)])
def test_smooth_frames_carry_int_delta_on_the_exponent_plane(name, plane):
    """The reference's smooth-data frames use the split chain with IntDelta on
    the exponent terminal (_chains.py:360-390, 581-600); the plan carries it
    as plane op 1 at byte width, on that plane only."""
    for path in sorted(glob.glob(os.path.join(FRAMES, name + "_*.body"))):
        plan, ents, _ = api.container_plan(PTWS + _read(path))
        assert ents[0].status == 0 and ents[0].plan_index == 0
        t = P.decode_plan(plan)[0]
        assert [(p.op, p.op_param) for p in t.planes] == [
            (P.PLANE_OP_INT_DELTA, 1) if i == plane else (P.PLANE_OP_NONE, 0) for i in range(len(t.planes))]


def test_reader_rejects_broken_files():
    good = _read(os.path.join(FILES, "legacy_v1_1_0.ptwm"))
    for bad in (b"", b"\x89PTWM", good[:-1], good[:90] + good[91:], b"\x89PTWQ" + good[5:]):
        with pytest.raises(NativeError) as ei:
            api.container_plan(bad)
        assert ei.value.rc == -1
    ptwc = _read(os.path.join(FILES, "ptwc_bound_source"))
    flipped = bytearray(ptwc)
    flipped[30] ^= 0x10  # inside the hashed metadata
    with pytest.raises(NativeError):
        api.container_plan(bytes(flipped))
    for name in ("regression_capacity_overflow", "regression_truncated_header_with_sentinel"):
        pass  # the reference's regression inputs: bad magic, rejected above as -1


@pytest.mark.parametrize("path", _legacy()[:3] + sorted(glob.glob(os.path.join(FILES, "ptwc_*"))),
                         ids=os.path.basename)
def test_reader_survives_truncation_and_bit_flips(path):
    """Every truncation and a spread of single-byte corruptions either parse
    or fail with -1: the reader never reads out of bounds (it runs in this
    process, so an overrun would crash the test run)."""
    data = _read(path)
    rng = np.random.default_rng(len(data))
    cuts = list(range(0, len(data), max(1, len(data) // 300)))
    for k in cuts:
        try:
            api.container_plan(data[:k])
        except NativeError as e:
            assert e.rc == -1
    for pos in rng.integers(0, len(data), 400):
        b = bytearray(data)
        b[pos] ^= int(rng.integers(1, 256))
        try:
            plan, ents, out_len = api.container_plan(bytes(b))
            P.decode_plan(plan)  # a plan the reader writes always parses
            for e in ents:
                assert e.status in (0, -1, -5)
        except NativeError as e:
            assert e.rc == -1


def test_plan_offsets_stay_inside_the_file():
    for path in _legacy() + sorted(glob.glob(os.path.join(FILES, "ptwc_*"))):
        data = _read(path)
        plan, _, out_len = api.container_plan(data)
        for t in P.decode_plan(plan):
            assert t.out_offset + t.out_len <= out_len
            for p in t.planes:
                assert p.payload_offset + p.payload_len <= len(data)


# ---- canonical forms and built-in ids ------------------------------------------------

def _frame_passthrough():
    """A one-tensor compact frame (bytes, passthrough chain, Identity plane)
    and the offset of its CW2 chain, whose canonical bytes are
    02 01 01 | 00 00 | 30 00 | 01 | 10 c7: two nodes (a bound Source, the
    byte passthrough), one edge on the implicit spine, one terminal (node 1,
    output 0, role Value { IntN { 8 } })."""
    raw = bytes(range(256))
    f = api.container_write([api.WriteTensor("x", 13, P.CHAIN_PASSTHROUGH, [256], [api.WritePlane(0, raw)])],
                            layout="frame")
    cw2 = bytes.fromhex("02010100003000" + "01" + "10c7")
    at = f.find(cw2)
    assert at > 0
    return f, at, len(cw2)


@pytest.mark.parametrize("what,chain", [
    ("spine edge written out", "02010100003000" + "00" + "0000010000" + "10c7"),
    ("terminal ref escaped needlessly", "02010100003000" + "01" + "ff0100c7"),
    ("reserved terminal ref byte", "02010100003000" + "01" + "f0c7"),
    ("role escaped needlessly", "02010100003000" + "01" + "10" + "ff010108"),
    ("invalid escaped role", "02010100003000" + "01" + "10" + "ff0405"),
])
def test_non_canonical_chain_wire_is_refused(what, chain):
    """chain/wire_compact.rs:339 (spine edge), :352 (terminal escape), the
    reserved terminal bytes, :528 (role escape) and Role::read's value checks
    (types/role.rs:283-291): the frame's chain is refused, so the frame is."""
    f, at, n = _frame_passthrough()
    api.container_plan(f)
    bad = f[:at] + bytes.fromhex(chain) + f[at + n:]
    with pytest.raises(Exception):
        api.container_plan(bad)


def test_escaped_role_without_a_code_is_read():
    """A role with no one-byte code (Value { IntN { 40 } }) is written
    escaped: the chain reads (the plane's role just has no decode plan)."""
    f, at, n = _frame_passthrough()
    ok = f[:at] + bytes.fromhex("02010100003000" + "01" + "10" + "ff010128") + f[at + n:]
    _, ents, _ = api.container_plan(ok)
    assert len(ents) == 1


def _ptwc_split(d):
    o = 11
    lens = []
    for _ in range(3):
        v = sh = 0
        while True:
            c = d[o]
            o += 1
            v |= (c & 0x7F) << sh
            sh += 7
            if not c & 0x80:
                break
        lens.append(v)
    hdr_end = o + 8
    et = d[hdr_end:hdr_end + lens[0]]
    pre = d[hdr_end + lens[0]:hdr_end + lens[0] + lens[1]]
    reg = d[hdr_end + lens[0] + lens[1]:hdr_end + sum(lens)]
    return d[:11], et, pre, reg, d[hdr_end + sum(lens):]


def _var(v):
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        out.append(b | (0x80 if v else 0))
        if not v:
            return bytes(out)


def _ptwc_join(head11, et, pre, reg, rest):
    """A compact container with new sections: the lengths and meta_xxh64
    (over the header up to it and the three sections, ptwc.rs) recomputed;
    records follow the registry, so the body is unchanged."""
    pre_hdr = head11 + _var(len(et)) + _var(len(pre)) + _var(len(reg))
    meta = O.xxh64(pre_hdr + et + pre + reg)
    return pre_hdr + meta.to_bytes(8, "little") + et + pre + reg + rest


def _with_entries(et, extra):
    n = et[0]
    assert n < 0x80
    return bytes([n + len(extra)]) + et[1:] + b"".join(extra)


def _builtin_id(name, version="1.1.0"):
    return O.blake3(b"\xbb" * 32 + b"\x00" + name.encode() + b"\x00" + version.encode())


def _full_entry(cid: bytes, label: str) -> bytes:
    lb = label.encode()
    e = cid + len(lb).to_bytes(2, "little") + lb + (2).to_bytes(2, "little") + (1).to_bytes(2, "little") + b"\x01\x02"
    e += (0).to_bytes(4, "little") + b"\x01" + (0).to_bytes(2, "little") + (0).to_bytes(2, "little") + bytes(16)
    return b"\x7f" + _var(len(e)) + e


def test_compact_table_named_and_full_entries():
    """extension/compact_table.rs:198-235: a built-in with a wire id stored by
    name, or a full entry carrying a built-in's id (current or, with its
    label, another version), is refused; the host-side built-ins by name and
    a third-party full entry are read."""
    d = open(os.path.join(FILES, "ptwc_trimmed"), "rb").read()
    head, et, pre, reg, rest = _ptwc_split(d)
    assert _ptwc_join(head, et, pre, reg, rest) == d  # the helpers rebuild the file
    good = [b"\x03" + _var(20) + b"classifier_heuristic",
            _full_entry(bytes(range(32)), "org.example.codec@1.0.0")]
    for e in good:
        _, ents, _ = api.container_plan(_ptwc_join(head, _with_entries(et, [e]), pre, reg, rest))
        assert ents
    bad = [b"\x03" + _var(7) + b"huffman",
           b"\x03" + _var(5) + b"bogus",
           _full_entry(_builtin_id("huffman"), "anything@1"),
           _full_entry(_builtin_id("zstd", "1.0.0"), "io.ptwm.builtin.zstd@1.0.0")]
    for e in bad:
        with pytest.raises(Exception):
            api.container_plan(_ptwc_join(head, _with_entries(et, [e]), pre, reg, rest))


def test_compact_prelude_reserved_and_padding_must_be_zero():
    """container.rs:1569-1580: the compact container's prelude is refused
    unless it is the one encoding of its entries (reserved field and name
    padding zero)."""
    d = open(os.path.join(FILES, "ptwc_trimmed"), "rb").read()
    head, et, pre, reg, rest = _ptwc_split(d)
    assert pre == b"\x00" * 4
    state = b"\x01\x02\x03"

    def entry(reserved=0, pad=b"\x00"):
        e = (7).to_bytes(2, "little") + (4).to_bytes(2, "little") + b"\x00\x01" + reserved.to_bytes(2, "little")
        e += O.xxh64(state).to_bytes(8, "little") + (3).to_bytes(2, "little") + b"abc" + pad
        return e + len(state).to_bytes(4, "little") + state

    ok = (1).to_bytes(4, "little") + entry()
    api.container_plan(_ptwc_join(head, et, ok, reg, rest))
    for p in ((1).to_bytes(4, "little") + entry(reserved=1), (1).to_bytes(4, "little") + entry(pad=b"\x01")):
        with pytest.raises(Exception):
            api.container_plan(_ptwc_join(head, et, p, reg, rest))


def test_legacy_builtin_entries_are_recognised_by_id():
    """A legacy entry is a built-in only by its id (the current version's, or
    its label's version derivation, extension/builtins.rs:302-332): with the
    plane codecs' ids changed and their labels kept, no tensor plans (all
    -5, codecs the device does not know) and the file still opens."""
    d = bytearray(open(os.path.join(FILES, "legacy_v1_1_0.ptwm"), "rb").read())
    et_off, et_len = (int.from_bytes(d[k:k + 8], "little") for k in (11, 19))
    count = int.from_bytes(d[et_off:et_off + 4], "little")
    o = et_off + 4
    flipped = 0
    for _ in range(count):  # flip a bit of every plane codec entry's canonical id
        ll = int.from_bytes(d[o + 32:o + 34], "little")
        if int.from_bytes(d[o + 34 + ll:o + 36 + ll], "little") == 2:  # Kind::PlaneCodec
            d[o] ^= 1
            flipped += 1
        p = o + 34 + ll + 6
        cl = int.from_bytes(d[p:p + 4], "little")
        p += 4 + cl + 1
        p += 2 + int.from_bytes(d[p:p + 2], "little")
        p += 2 + int.from_bytes(d[p:p + 2], "little")
        o = p + 16
    assert o == et_off + et_len and flipped > 0
    d[27:59] = O.blake3(bytes(d[et_off:et_off + et_len]))
    _, ents, _ = api.container_plan(bytes(d))
    assert ents and all(e.plan_index == -1 and e.status == -5 for e in ents), [e.status for e in ents]


def _legacy_plane_state_at(data: bytes, payload_off: int, payload_len: int, rows: bool = False) -> int:
    """File offset of a legacy plane record's state_source byte, found back
    from its payload (plane_record.rs:110-272: role, flags, codec, table
    index, state_source, state_version, state_info u16, inline length u32,
    payload_len u64, CRC u32, layout u8 [row_len u32], payload) for an
    unchunked plane with a CRC and no inline state."""
    import struct

    o = payload_off - 1 - (4 if rows else 0) - 4 - 8
    if struct.unpack_from("<Q", data, o)[0] != payload_len or struct.unpack_from("<I", data, o - 4)[0] != 0:
        return None  # another record shape (rows layout, inline state)
    return o - 8


def _prelude_mask_at(data: bytes, state_off: int) -> int:
    """File offset of the applies_to_mask byte of the prelude entry whose state starts at state_off
    (prelude.rs write_prelude: id, codec, version, mask, reserved, xxh64,
    name_len, name, pad to 4, state_len, state)."""
    import struct

    for n in range(64):
        pad = (4 - n % 4) % 4
        e = state_off - 4 - pad - n - 18
        if e >= 0 and struct.unpack_from("<H", data, e + 16)[0] == n and \
                struct.unpack_from("<H", data, e + 2)[0] == O.CODEC_O1SAC:
            return e + 5
    raise AssertionError("prelude entry not found")


def test_shared_state_of_a_stateless_codec_is_checked_then_ignored():
    """container.rs:2051-2100 resolves an unchunked plane's shared state
    whatever its codec (entry present, same version, role covered by
    applies_to_mask, stored xxh64); a codec without state then ignores it
    (codecs/zstd.rs:65-106 and the like).  Planes of legacy_v1_1_0.ptwm
    patched to name the file's Order1ScaleAC prelude entry plan and decode
    as before when the checks pass, and are refused (-1) when they fail."""
    name = "legacy_v1_1_0.ptwm"
    data = open(os.path.join(FILES, name), "rb").read()
    plan, ents, out_len = api.container_plan(data)
    ts = P.decode_plan(plan)
    want = plan_oracle.decode_plan(data, plan, out_len)
    scale = [(e, ts[e.plan_index]) for e in ents if e.name.endswith(".scale")][0][1].planes[0]
    s_off, _, _, s_ver = scale.state
    o1 = _legacy_plane_state_at(data, scale.payload_offset, scale.payload_len, rows=True)
    assert o1 is not None and data[o1] == 2  # the scale plane names its prelude entry
    sid = data[o1 + 2] | (data[o1 + 3] << 8)
    mask_at = _prelude_mask_at(data, s_off)
    cases, accepted = 0, 0
    for e in ents:
        t = ts[e.plan_index]
        for p in t.planes:
            if p.codec == O.CODEC_O1SAC or p.chunks:
                continue
            at = _legacy_plane_state_at(data, p.payload_offset, p.payload_len)
            if at is None:
                continue
            role = data[at - 6]
            for mask, ver, ident in ((data[mask_at], s_ver, sid), (0xFF, s_ver, sid), (0xFF, s_ver + 1, sid),
                                     (0xFF, s_ver, sid + 7)):
                ok = ver == s_ver and ident == sid and (not 1 <= role <= 8 or bool(mask >> (role - 1) & 1))
                b = bytearray(data)
                b[mask_at] = mask  # the entry's stored xxh64 covers its state bytes only
                b[at] = 2
                b[at + 1] = ver
                b[at + 2:at + 4] = ident.to_bytes(2, "little")
                plan2, ents2, out2 = api.container_plan(bytes(b))
                e2 = [x for x in ents2 if x.name == e.name][0]
                if ok:
                    assert e2.status == 0, (e.name, role)
                    got = plan_oracle.decode_plan(bytes(b), plan2, out2)
                    assert got[e2.out_offset:e2.out_offset + e2.orig_size] == \
                        want[e.out_offset:e.out_offset + e.orig_size]
                    accepted += 1
                else:
                    assert e2.status == -1, (e.name, role, ver, ident)
                cases += 1
    assert cases >= 12 and accepted >= 3
