"""Sanitized fuzzing of the parsers of untrusted bytes, on the CPU.

tests/fuzz/fuzz_parsers.cpp is a libFuzzer target over the container reader
(ptwm_mi355x_container_plan: legacy, PTWC, PTWS) and the decode-plan parser
(parse_plan), built for the host with AddressSanitizer and
UndefinedBehaviorSanitizer by tests/fuzz/Makefile (no device code).  The
seeds are the reference's golden files and the plans read from them; the
run must end without a sanitizer report, a crash or a broken invariant (a
plan the reader writes always parses; a file the rewriter writes rewrites to
itself).
"""
import glob
import os
import shutil
import struct
import subprocess

import pytest

from ptwm_amd import api

HERE = os.path.dirname(os.path.abspath(__file__))
FUZZ = os.path.join(HERE, "fuzz")
CLANG = "/opt/rocm/llvm/bin/clang++"


def _seeds(d):
    k = 0
    for p in sorted(glob.glob(os.path.join(HERE, "golden", "ptwm_files", "*"))):
        data = open(p, "rb").read()
        open(os.path.join(d, "f%03d" % k), "wb").write(b"\x00" + data)
        open(os.path.join(d, "g%03d" % k), "wb").write(b"\x02" + data)
        plan, _, _ = api.container_plan(data)
        open(os.path.join(d, "p%03d" % k), "wb").write(b"\x01" + plan)
        k += 1
    for p in sorted(glob.glob(os.path.join(HERE, "golden", "ptws_frames", "*.body"))):
        frame = b"\x89PTWS" + open(p, "rb").read()
        open(os.path.join(d, "s%03d" % k), "wb").write(b"\x00" + frame)
        open(os.path.join(d, "w%03d" % k), "wb").write(b"\x02" + frame)
        plan, _, _ = api.container_plan(frame)  # plans with plane ops (the smooth frames)
        open(os.path.join(d, "q%03d" % k), "wb").write(b"\x01" + plan)
        k += 1
    # regressions: a legacy record whose name runs past the record's end;
    # inputs the fuzzer found (tests/golden/fuzz_regress, with their mode byte)
    open(os.path.join(d, "r000"), "wb").write(b"\x00" + overlong_name_file())
    for k, p in enumerate(sorted(glob.glob(os.path.join(HERE, "golden", "fuzz_regress", "*.bin")))):
        shutil.copy(p, os.path.join(d, "x%03d" % k))


def overlong_name_file() -> bytes:
    """legacy_v1_1_0.ptwm with its first record's name length (the u16 at
    record offset 16, tensor_record.rs:265-420) set to the record's length,
    so that the name runs past the record's end."""
    data = bytearray(open(os.path.join(HERE, "golden", "ptwm_files", "legacy_v1_1_0.ptwm"), "rb").read())
    _, ents, _ = api.container_plan(bytes(data))
    e = ents[0]
    assert struct.unpack_from("<H", data, e.record_offset + 16)[0] == len(e.name.encode())
    struct.pack_into("<H", data, e.record_offset + 16, e.record_len)
    return bytes(data)


def test_overlong_legacy_name_is_rejected():
    """The record is listed as invalid (-1, no name reported); the other
    records still plan."""
    _, ents, _ = api.container_plan(overlong_name_file())
    assert ents[0].status == -1 and ents[0].plan_index == -1 and ents[0].name == ""
    assert all(e.status == 0 for e in ents[1:])


def test_chunk_offset_past_the_payload_is_rejected():
    """A legacy file the fuzzer derived from legacy_v1_1_0.ptwm: the chunk
    table of the last tensor's first plane starts past the plane's payload.
    The reference refuses the record at decode (container.rs:1998-2009);
    the reader lists it invalid (-1, not planned) instead of writing a plan
    whose chunk table leaves the payload, and the other records still plan."""
    data = open(os.path.join(HERE, "golden", "fuzz_regress", "legacy_chunk_offset_past_payload.bin"), "rb").read()
    assert data[0] == 0  # fuzz mode byte: the container reader
    plan, ents, _ = api.container_plan(data[1:])
    assert ents[-1].status == -1 and ents[-1].plan_index == -1
    assert sum(e.plan_index >= 0 for e in ents) == 4


@pytest.mark.skipif(not os.path.exists(CLANG), reason="ROCm clang (libFuzzer) not installed")
def test_parsers_survive_sanitized_fuzzing(tmp_path):
    r = subprocess.run(["make", "-s", "-C", FUZZ], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    corpus = tmp_path / "corpus"
    corpus.mkdir()
    _seeds(str(corpus))
    exe = os.path.join(FUZZ, "_build", "fuzz_parsers")
    r = subprocess.run([exe, "-max_total_time=25", "-seed=7", "-max_len=65536", "-rss_limit_mb=4096",
                        "-artifact_prefix=" + str(tmp_path) + "/", str(corpus)],
                       capture_output=True, text=True, timeout=300, cwd=str(tmp_path))
    tail = "\n".join(r.stderr.splitlines()[-25:])
    assert r.returncode == 0, tail
    assert "Done" in r.stderr
    shutil.rmtree(corpus, ignore_errors=True)
