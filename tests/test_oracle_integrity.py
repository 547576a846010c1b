"""The oracle's integrity functions, pinned.

- XXH64 (seed 0): the reference's own golden table (legacy_fixtures.rs:63-123,
  decoded length + xxh64 of nine tensors, whose inputs the fixture's SplitMix64
  generator reproduces) and the xxhash module (XXH 0.8.2) on random inputs of
  every length class (< 4, < 8, < 32 bytes, stripes + tails).
- CRC-32/ISO-HDLC: zlib.crc32 (the same polynomial, init and final xor as
  crc32fast 1.5.0) and the catalogue check value crc("123456789") = 0xCBF43926.
"""
import os
import sys
import zlib

import numpy as np
import pytest

import oracle as O

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import legacy_tensors as G  # noqa: E402


def test_xxh64_matches_reference_golden_table():
    t = G.tensors()
    for name, (n, h) in G.expected().items():
        assert len(t[name]) == n, name
        assert O.xxh64(t[name]) == h, name


LENS = list(range(0, 70)) + [127, 128, 129, 1000, 4096, 65537]


@pytest.mark.parametrize("n", LENS)
def test_xxh64_matches_xxhash_module(n):
    xxhash = pytest.importorskip("xxhash")
    d = np.random.default_rng(n).integers(0, 256, n, dtype=np.uint8).tobytes()
    assert O.xxh64(d) == xxhash.xxh64_intdigest(d, seed=0)
    assert O.xxh64(d, 12345) == xxhash.xxh64_intdigest(d, seed=12345)


def test_crc32_check_value_and_zlib():
    assert O.crc32(b"123456789") == 0xCBF43926
    for n in LENS:
        d = np.random.default_rng(1000 + n).integers(0, 256, n, dtype=np.uint8).tobytes()
        assert O.crc32(d) == zlib.crc32(d), n
    # streaming form: crc(a + b) from crc(a)
    a, b = b"plane-", b"bytes"
    assert O.crc32(b, O.crc32(a)) == zlib.crc32(a + b)
