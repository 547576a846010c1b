"""Reference files decoded on the GPU, and the tANS device decoder.

The reference's golden containers and frames (tests/golden/ptwm_files,
tests/golden/ptws_frames: its legacy fixtures, PTWC corpus and PTWS corpus)
are read by ptwm_mi355x_container_plan, copied to the device as they are,
and restored by one ptwm_hardware_backend_v1_dispatch_decode_cuda call with
the plane CRC-32s and payload hashes the files carry checked on the way.
Every planned tensor must equal the oracle's decode of the same plan and,
for the legacy fixtures, the EXPECTED XXH64 of legacy_fixtures.rs:63-123.

tANS (entropy/tans/mod.rs, codecs/tans.rs): payloads written by the oracle's
restatement (itself pinned by the fixtures' chunked tensor on CPU) decode on
the device bit-exactly, whole and in chunk frames, and malformed ones are
InvalidInput (-1).
"""
import glob
import json
import os
import sys

import numpy as np
import pytest

import oracle as O
from ptwm_amd import api, ids, plan as P

import plan_oracle

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

HERE = os.path.dirname(os.path.abspath(__file__))
FILES = os.path.join(HERE, "golden", "ptwm_files")
FRAMES = os.path.join(HERE, "golden", "ptws_frames")
EXPECTED = json.load(open(os.path.join(HERE, "golden", "legacy_xxh64.json")))
TANS_ID = "e4868545e7b22282695972441494e70569ab27595d19349114e852125d96daa4"


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dev_bytes(b: bytes):
    t = torch.empty(max(1, len(b)), dtype=torch.uint8, device="cuda:0")
    if b:
        t[: len(b)].copy_(torch.from_numpy(np.frombuffer(b, np.uint8).copy()))
    return t[: len(b)]


def dispatch(state: bytes, src, out) -> int:
    n = api.hardware_backend_dispatch_decode_cuda(ids.HARDWARE_BACKEND_LABEL, ids.DECODE_PLAN_LABEL, state, src, out, 0)
    torch.cuda.synchronize()
    return n


def _inputs():
    for p in sorted(glob.glob(os.path.join(FILES, "*"))):
        yield os.path.basename(p), open(p, "rb").read()
    for p in sorted(glob.glob(os.path.join(FRAMES, "*.body"))):
        yield os.path.basename(p), b"\x89PTWS" + open(p, "rb").read()


INPUTS = list(_inputs())


@pytest.mark.parametrize("name,data", INPUTS, ids=[n for n, _ in INPUTS])
def test_reference_file_decodes_on_device(name, data):
    plan, ents, out_len = api.container_plan(data)
    n_planned = sum(e.plan_index >= 0 for e in ents)
    note(f"container {name}: {len(ents)} tensors, {n_planned} planned, out {out_len} B")
    assert n_planned > 0, "every golden file has tensors the device restores"
    want = plan_oracle.decode_plan(data, plan, out_len)
    src = dev_bytes(data)
    out = torch.full((out_len,), 0xA5, dtype=torch.uint8, device="cuda:0")
    assert dispatch(plan, src, out) == sum(e.orig_size for e in ents if e.plan_index >= 0)
    got = out.cpu().numpy().tobytes()
    for e in ents:
        if e.plan_index < 0:
            continue
        raw = got[e.out_offset:e.out_offset + e.orig_size]
        assert raw == want[e.out_offset:e.out_offset + e.orig_size], e.name
        if e.name in EXPECTED:
            assert "%016x" % O.xxh64(raw) == EXPECTED[e.name][1]


def test_legacy_chunked_tans_tensor_matches_expected():
    data = open(os.path.join(FILES, "legacy_v1_1_0.ptwm"), "rb").read()
    plan, ents, out_len = api.container_plan(data)
    e = [x for x in ents if x.name == "model.layers.2.chunked.weight"][0]
    t = P.decode_plan(plan)[e.plan_index]
    t.out_offset = 0
    src = dev_bytes(data)
    out = torch.zeros(e.orig_size, dtype=torch.uint8, device="cuda:0")
    assert dispatch(P.encode_plan([t]), src, out) == 1024
    assert "%016x" % O.xxh64(out.cpu().numpy().tobytes()) == EXPECTED["model.layers.2.chunked.weight"][1]
    # the file's own CRC of the tANS plane and its payload hash are checked
    t.planes[1].crc32 ^= 1
    with pytest.raises(Exception) as ei:
        dispatch(P.encode_plan([t]), src, out)
    assert getattr(ei.value, "rc", None) == -1


def _tans_planes():
    rng = np.random.default_rng(11)
    yield "geom-64k", (rng.geometric(0.25, 65536) % 256).astype(np.uint8)
    yield "normal-300k", np.clip(rng.normal(120, 9, 300_001), 0, 255).astype(np.uint8)
    yield "two-sym", rng.integers(0, 2, 4097).astype(np.uint8) * 200
    yield "uniform-raw", rng.integers(0, 256, 5000, dtype=np.uint8)   # stored raw (tag 0)
    yield "const", np.full(777, 9, np.uint8)                            # one symbol: raw
    yield "tiny", np.array([1, 2, 1], np.uint8)


TP = list(_tans_planes())


@pytest.mark.parametrize("name,plane", TP, ids=[n for n, _ in TP])
def test_tans_payloads_decode_bit_exact(name, plane):
    note(f"tans {name} n={plane.size}")
    whole = O.codec_encode(O.CODEC_TANS, plane)
    chunked, ent = O.encode_plane_chunked(O.CODEC_TANS, plane, 16384)
    data = whole + b"\x00" * 3 + chunked          # the chunked payload at an odd offset
    off2 = len(whole) + 3
    n = plane.size
    tensors = [P.TensorPlan(P.CHAIN_PASSTHROUGH, 0, n, [P.PlanePlan(O.CODEC_TANS, 0, len(whole), n)]),
               P.TensorPlan(P.CHAIN_PASSTHROUGH, (n + 255) // 256 * 256, n,
                            [P.PlanePlan(O.CODEC_TANS, off2, len(chunked), n, [tuple(e) for e in ent])])]
    out_len = tensors[1].out_offset + n
    src = dev_bytes(data)
    out = torch.zeros(max(out_len, 1), dtype=torch.uint8, device="cuda:0")
    assert dispatch(P.encode_plan(tensors), src, out) == 2 * n
    got = out.cpu().numpy()
    assert np.array_equal(got[:n], plane)
    assert np.array_equal(got[tensors[1].out_offset:tensors[1].out_offset + n], plane)


def _tans_top_word(payload):
    """Index of the stream word holding the last coded bit (the decoder
    stages the stream in pieces of 1024 words from the end down)."""
    enc = payload[5:]
    nsym = enc[1] | (enc[2] << 8)
    off = 3 + 3 * nsym + 8
    tb = int.from_bytes(enc[off - 8:off], "little")
    return (tb - 1) >> 5


@pytest.mark.parametrize("edge", [0, 1, 2])
def test_tans_streams_whose_last_words_straddle_a_stage_piece(edge):
    """The decoder reads the top word, the one below and the next one before
    the first symbol: streams whose top word is the first, second or third
    of a 1024-word piece restage on one of those reads."""
    rng = np.random.default_rng(40 + edge)
    base = np.clip(rng.normal(120, 20, 200_000), 0, 255).astype(np.uint8)
    # h bits per symbol on average: aim at the piece edge, then walk outwards
    n0 = 150_000
    h = 32 * _tans_top_word(O.codec_encode(O.CODEC_TANS, base[:n0])) / n0
    aim = int((32 * (1024 * 29 + edge) + 16) / h)
    found = None
    for d in range(400):
        for n in (aim + d, aim - d):
            pay = O.codec_encode(O.CODEC_TANS, base[:n])
            top = _tans_top_word(pay)
            if top % 1024 == edge:
                found = n
                break
        if found:
            break
    assert found, "no prefix length puts the top word at the piece edge"
    n = found
    note(f"tans stage edge {edge}: n={n} top word {top}")
    plane = base[:n]
    t = P.TensorPlan(P.CHAIN_PASSTHROUGH, 0, n, [P.PlanePlan(O.CODEC_TANS, 0, len(pay), n)])
    out = torch.zeros(n, dtype=torch.uint8, device="cuda:0")
    assert dispatch(P.encode_plan([t]), dev_bytes(pay), out) == n
    assert np.array_equal(out.cpu().numpy(), plane)


def test_tans_planes_of_a_bf16_tensor():
    w = (torch.randn(1000, 1500, generator=torch.Generator().manual_seed(2)) * 0.02).to(torch.bfloat16)
    data = w.view(torch.uint8).reshape(-1).numpy().tobytes()
    planes = O.chain_forward(P.CHAIN_IEEE16_SPLIT2, data)
    pays = [O.codec_encode(O.CODEC_TANS, p) for p in planes]
    t = P.TensorPlan(P.CHAIN_IEEE16_SPLIT2, 0, len(data), [
        P.PlanePlan(O.CODEC_TANS, 0, len(pays[0]), len(planes[0]), crc32=O.crc32(planes[0])),
        P.PlanePlan(O.CODEC_TANS, len(pays[0]), len(pays[1]), len(planes[1]), crc32=O.crc32(planes[1]))],
        xxh64=O.xxh64(data))
    src = dev_bytes(pays[0] + pays[1])
    out = torch.zeros(len(data), dtype=torch.uint8, device="cuda:0")
    assert dispatch(P.encode_plan([t]), src, out) == len(data)
    assert out.cpu().numpy().tobytes() == data


def test_tans_single_plane_entry_point_and_rejections():
    plane = (np.random.default_rng(5).geometric(0.3, 20000) % 256).astype(np.uint8)
    pay = O.codec_encode(O.CODEC_TANS, plane)
    assert pay[0] == 1
    src = dev_bytes(pay)
    out = torch.zeros(plane.size, dtype=torch.uint8, device="cuda:0")
    n = api.plane_codec_decode_cuda(ids.PLANE_CODEC_LABEL, TANS_ID, b"", src, out, 0)
    torch.cuda.synchronize()
    assert n == plane.size and np.array_equal(out.cpu().numpy(), plane)
    # corruptions the reference rejects: each is InvalidInput on the device
    nsym = pay[6] | (pay[7] << 8)
    tb = 5 + 3 + 3 * nsym
    bad = []
    b = bytearray(pay); b[5] = 12; bad.append(b)                       # table_log
    b = bytearray(pay); b[9] ^= 1; bad.append(b)                       # frequencies off L
    b = bytearray(pay); bits = int.from_bytes(b[tb:tb + 8], "little")
    b[tb:tb + 8] = (bits + 1).to_bytes(8, "little"); bad.append(b)     # trailing bit
    b = bytearray(pay); b[-1] ^= 0x01; bad.append(b)                   # a stream bit
    for k, b in enumerate(bad):
        assert _oracle_rejects(bytes(b), plane.size), k
        t = P.TensorPlan(P.CHAIN_PASSTHROUGH, 0, plane.size, [P.PlanePlan(O.CODEC_TANS, 0, len(b), plane.size)])
        with pytest.raises(Exception) as ei:
            dispatch(P.encode_plan([t]), dev_bytes(bytes(b)), out)
        assert getattr(ei.value, "rc", None) == -1, k


def _oracle_rejects(payload, n):
    try:
        got = O.codec_decode(O.CODEC_TANS, payload, n)
    except O.OracleError:
        return True
    return len(got) != n
