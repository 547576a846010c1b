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
