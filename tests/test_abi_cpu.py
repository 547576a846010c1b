"""CPU checks of the boundary: the C-ABI library loads, exports every symbol
include/ptwm_mi355x.h declares, and its canonical ids are the blake3
derivations of extension/id.rs:21-30 (recomputed with the oracle's blake3,
itself pinned by the built-in ids found in the reference's legacy .ptwm
fixtures).  No compute call is made here (no GPU)."""
import ctypes as C
import os
import re

import pytest

from ptwm_amd import _native, ids, plan

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    txt = open(os.path.join(ROOT, "include", "ptwm_mi355x.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(ptwm_[a-z0-9_]+)\s*\(", txt)))


def test_library_exports_every_declared_symbol():
    L = _native.lib()
    syms = header_symbols()
    assert len(syms) >= 12
    for s in syms:
        assert hasattr(L, s), s
    assert sorted(_native.symbol_names()) == syms


def test_reference_loader_symbol_set_complete():
    # native.rs:239-273 requires encode+decode and all-or-none of the 3 CUDA symbols
    L = _native.lib()
    for s in ("ptwm_plane_codec_v1_encode", "ptwm_plane_codec_v1_decode", "ptwm_plane_codec_v1_decode_stateful",
              "ptwm_plane_codec_v1_encode_cuda", "ptwm_plane_codec_v1_decode_cuda",
              "ptwm_plane_codec_v1_cuda_stream_handle", "ptwm_hardware_backend_v1_cuda_stream_handle",
              "ptwm_hardware_backend_v1_dispatch_decode_cuda"):
        assert hasattr(L, s)


def test_abi_version_and_ids(orc):
    L = _native.lib()
    assert L.ptwm_mi355x_abi_version() == 1
    out = (C.c_uint8 * 32)()
    for which, label in enumerate([ids.PLANE_CODEC_LABEL, ids.HARDWARE_BACKEND_LABEL, ids.DECODE_PLAN_LABEL,
                                   ids.RANS_CODEC_LABEL]):
        assert L.ptwm_mi355x_canonical_id(which, out) == 0
        want = orc.blake3(bytes(32) + b"\x00" + label.encode() + b"\x00" + ids.OWN_VERSION.encode())
        assert bytes(out) == want == bytes.fromhex(ids.OWN_IDS[label])
    assert L.ptwm_mi355x_canonical_id(7, out) == -1


def test_builtin_ids_are_blake3_derivations(orc):
    for (name, ver), hx in ids.BUILTIN_IDS.items():
        assert orc.blake3(bytes([0xBB] * 32) + b"\x00" + name.encode() + b"\x00" + ver.encode()).hex() == hx


def test_builtin_ids_appear_in_reference_fixture_bytes():
    """The legacy container fixtures intern the built-in ids in their
    Extension Table (tests/fixtures/legacy_v1_1_0.ptwm); checked via the
    committed copy of those 32-byte ids under tests/golden."""
    import json
    g = json.load(open(os.path.join(ROOT, "tests", "golden", "builtin_ids_in_fixtures.json")))
    for entry in g:
        assert ids.BUILTIN_IDS[(entry["name"], entry["version"])] == entry["id"]


def test_resolve_selector():
    assert ids.resolve_codec_selector("huffman").hex() == ids.BUILTIN_IDS[("huffman", "1.1.0")]
    assert ids.resolve_codec_selector("blake3:" + "ab" * 32) == bytes([0xAB] * 32)
    assert ids.codec_wire_id(ids.resolve_codec_selector("rans")) == ids.CODEC_RANS
    with pytest.raises(LookupError):
        ids.resolve_codec_selector("nope")


def test_unknown_codec_id_is_unsupported_without_touching_device():
    L = _native.lib()
    bad = bytes(32)
    assert L.ptwm_plane_codec_v1_decode_cuda(1, None, 0, bad, 32, 0, 0, 0, 0, 0) == -5
    assert L.ptwm_plane_codec_v1_decode_cuda(1, None, 0, bad, 31, 0, 0, 0, 0, 0) == -5
    assert L.ptwm_hardware_backend_v1_dispatch_decode_cuda(1, None, 0, bad, 32, 0, 0, 0, 0, 0) == -5
    huf = bytes.fromhex(ids.BUILTIN_IDS[("huffman", "1.1.0")])
    assert L.ptwm_plane_codec_v1_decode_cuda(1, b"x", 1, huf, 32, 0, 0, 0, 0, 0) == -1   # state rejected


def test_plan_roundtrip_and_validation():
    t = plan.TensorPlan(plan.CHAIN_IEEE16_SPLIT2, 0, 64, [
        plan.PlanePlan(0, 0, 32, 32),
        plan.PlanePlan(1, 32, 20, 32, chunks=[(0, 16), (10, 16)], crc32=5),
    ])
    b = plan.encode_plan([t])
    back = plan.decode_plan(b)
    assert back[0].planes[1].chunks == [(0, 16), (10, 16)] and back[0].planes[1].crc32 == 5
    L = _native.lib()
    pid = bytes.fromhex(ids.OWN_IDS[ids.DECODE_PLAN_LABEL])
    # out buffer too small for the tensor: rejected on the host before any device work
    assert L.ptwm_hardware_backend_v1_dispatch_decode_cuda(1, b, len(b), pid, 32, 1 << 20, 52, 1 << 24, 63, 0) == -1
    # malformed plan
    assert L.ptwm_hardware_backend_v1_dispatch_decode_cuda(1, b[:-1], len(b) - 1, pid, 32, 1 << 20, 52, 1 << 24, 64, 0) == -1
