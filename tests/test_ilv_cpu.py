"""CPU checks of the huff_ilv codec (this build's GPU-native plane codec)
and of the product's host-side Huffman table builder.

huff_ilv has no reference counterpart: its wire format is specified by the
oracle's por_ilv_encode / por_ilv_decode.  What pins it: round trips over
edge sizes and distributions; its code lengths are exactly the reference
Huffman's (checked against the oracle restatement of tree.rs, itself pinned
in test_oracle_entropy.py); and its block / lane layout is checked from the
bytes (offset table, lane word counts, bit order) independently of the
decoder.
"""
import ctypes as C
import struct

import numpy as np
import pytest

import oracle as O
from ptwm_amd import _native


@pytest.mark.parametrize("seed", range(60))
def test_product_code_lengths_match_reference_restatement(orc, seed):
    rng = np.random.default_rng(seed)
    f = np.zeros(256, np.uint32)
    k = int(rng.integers(1, 257))
    syms = rng.choice(256, k, replace=False)
    kind = seed % 4
    if kind == 0:
        f[syms] = rng.integers(1, 1000, k)
    elif kind == 1:
        f[syms] = rng.integers(1, 4, k)             # many ties
    elif kind == 2:
        f[syms] = (2.0 ** rng.integers(0, 30, k)).astype(np.uint64).clip(1, 2**31)  # deep trees -> length limit
    else:
        f[syms] = rng.geometric(0.2, k) * 1000
    want = O.huf_lengths(f)
    got = np.zeros(256, np.uint8)
    rc = _native.lib().ptwm_mi355x_huffman_code_lengths(f.ctypes.data_as(C.c_void_p), got.ctypes.data_as(C.c_void_p))
    assert rc == 0
    assert np.array_equal(got, want)


def test_product_code_lengths_edge_cases(orc):
    L = _native.lib()
    got = np.zeros(256, np.uint8)
    z = np.zeros(256, np.uint32)
    assert L.ptwm_mi355x_huffman_code_lengths(z.ctypes.data_as(C.c_void_p), got.ctypes.data_as(C.c_void_p)) == -1
    f = np.zeros(256, np.uint32)
    a, b = 1, 1
    for i in range(30):                      # Fibonacci weights: depth 29 before limiting
        f[i] = a
        a, b = b, a + b
    assert L.ptwm_mi355x_huffman_code_lengths(f.ctypes.data_as(C.c_void_p), got.ctypes.data_as(C.c_void_p)) == 0
    assert np.array_equal(got, O.huf_lengths(f)) and got.max() == 11


def ilv_cases():
    rng = np.random.default_rng(3)
    for n in (0, 1, 2, 15, 16, 17, 1023, 1024, 1025, 16383, 16384, 16385, 40000):
        yield n, rng.geometric(0.3, n).clip(0, 255).astype(np.uint8).tobytes()
    yield 5000, bytes([9]) * 5000
    yield 70000, rng.integers(0, 16, 70000).astype(np.uint8).tobytes()
    yield 4096, rng.integers(0, 256, 4096).astype(np.uint8).tobytes()
    yield 50001, (15 - rng.geometric(0.45, 50001).clip(1, 16) + 1).astype(np.uint8).tobytes()  # skewed nibbles
    yield 3000, bytes([7]) * 3000                                                              # one nibble symbol


@pytest.mark.parametrize("n,src", list(ilv_cases()))
def test_ilv_spec_roundtrip(orc, n, src):
    p = O.ilv_encode(src)
    assert O.ilv_decode(p, n) == src


def test_ilv_layout_from_bytes(orc):
    """Parse a payload by hand: header, weights, offset table, lane word
    counts; re-derive lane 5's first group from its bits with the canonical
    codes (rev codes from the reference table restatement)."""
    rng = np.random.default_rng(9)
    n = 40000
    src = rng.geometric(0.4, n).clip(0, 40).astype(np.uint8).tobytes()
    p = O.ilv_encode(src)
    assert p[0] == 1 and struct.unpack_from("<I", p, 1)[0] == n
    w, wl = O.huf_decode_weights(p[5:])
    L = np.zeros(256, np.uint8)
    L[: len(w)] = np.frombuffer(w, np.uint8)
    assert np.array_equal(L, O.huf_lengths(O.histogram(src)))
    head = 5 + wl + (-(5 + wl)) % 4
    nb = -(-n // 16384)
    offs = struct.unpack_from(f"<{nb + 1}I", p, head)
    data0 = head + 4 * (nb + 1)
    assert offs[0] == 0 and offs[-1] == len(p) - data0
    _, _, rev = O.huf_table(L)
    for b in range(nb):
        blk = p[data0 + offs[b]: data0 + offs[b + 1]]
        counts = list(blk[:64])
        assert 64 + 4 * sum(counts) == len(blk)
        # lane 5: groups 5, 69, 133, ...; its first 16 symbols start at bit 0 of its words
        j = 5
        start = 64 + 4 * sum(counts[:j])
        words = blk[start: start + 4 * counts[j]]
        bits = int.from_bytes(words, "little")
        pos = 0
        g0 = b * 16384 + 16 * j
        for k in range(g0, min(g0 + 16, n)):
            s = src[k]
            code = int(rev[s])
            assert (bits >> pos) & ((1 << int(L[s])) - 1) == code
            pos += int(L[s])


def test_ilv_stored_when_not_beneficial(orc):
    src = np.random.default_rng(1).integers(0, 256, 3000).astype(np.uint8).tobytes()
    assert O.ilv_encode(src) == b"\x00" + src
    assert O.ilv_encode(b"") == b"\x00"


def test_ilv_decoder_rejects_corruption(orc):
    src = np.random.default_rng(2).geometric(0.3, 20000).clip(0, 255).astype(np.uint8).tobytes()
    p = bytearray(O.ilv_encode(src))
    bad = p[:]
    bad[len(bad) - 3] ^= 0x5A      # payload bits: decodes (wrong) or rejects, never crashes
    try:
        assert O.ilv_decode(bytes(bad), 20000) != src
    except O.OracleError:
        pass
    cut = bytes(p[:-4])
    with pytest.raises(O.OracleError):
        O.ilv_decode(cut, 20000)


def _kraft(lengths):
    return sum(2.0 ** -int(l) for l in lengths if l)


@pytest.mark.parametrize("seed", range(40))
def test_ilv_length_policy(orc, seed):
    """huff_ilv code lengths: the reference tree with the length limit 6 for
    alphabets of symbols < 16 (every pair of codes then fits one 12-bit
    decode lookup), else the reference's 11.  Checked by properties that do
    not restate the clamp: the limit holds, the code stays a prefix code,
    and a histogram whose tree already fits keeps the plain Huffman lengths
    (pinned by the optimality tests of the reference restatement)."""
    rng = np.random.default_rng(1000 + seed)
    f = np.zeros(256, np.uint32)
    nibble = seed % 2 == 0
    k = int(rng.integers(1, 17 if nibble else 257))
    syms = rng.choice(16 if nibble else 256, k, replace=False)
    f[syms] = (2.0 ** rng.uniform(0, 24, k)).astype(np.uint64).clip(1, 2**31)
    got = O.ilv_lengths(f)
    plain = O.huf_lengths(f)
    limit = 6 if nibble else 11
    assert got.max() <= limit and _kraft(got) <= 1.0 + 1e-12
    assert np.array_equal(got > 0, f > 0)
    if plain.max() <= limit:
        assert np.array_equal(got, plain)
    assert np.array_equal(got, O.huf_lengths_limited(f, limit))


def test_ilv_nibble_limit_on_fp8_exponent_histogram(orc):
    """The E4M3 exponent-nibble histogram of config 3 (per-row absmax N(0,1)):
    the 6-bit limit codes it no larger than the reference's 11-bit limit."""
    p = [0.00011, 0.00011, 0.00022, 0.00042, 0.00085, 0.00172, 0.00343, 0.00683, 0.01374, 0.0274, 0.05453,
         0.10744, 0.20101, 0.30964, 0.24284, 0.02971]
    f = np.zeros(256, np.uint32)
    f[:16] = np.round(np.array(p) * 1e7).astype(np.uint32)
    lim = O.ilv_lengths(f)
    ref = O.huf_lengths(f)
    assert ref.max() == 11 and lim.max() <= 6
    assert (f * lim.astype(np.uint64)).sum() <= (f * ref.astype(np.uint64)).sum()
