"""The rans_ilv specification (oracle por_rans_ilv_encode/decode), pinned.

rans_ilv is this library's own GPU-parallel rANS plane codec (no reference
counterpart), so its specification is pinned by what the mathematics and
the written layout fix rather than by reference vectors:
- a payload assembled by hand from the written layout decodes as specified;
- the frequency header is the reference's normalisation (rans/compress.rs
  normalize_freqs, pinned by its own known answers in test_oracle_entropy);
- rANS is an entropy coder: each lane's state grows by log2(2048 / f) per
  symbol (to within log2(33/32)) and sheds 16 bits per word, so a block's
  words and final states account for the symbols' cost;
- decode(encode(x)) == x over many distributions, including block tails;
- corruptions are rejected (word count, pad, final states).
"""
import math
import struct

import numpy as np
import pytest

import oracle as O

BLOCK = 16384


def _parse(p):
    n = struct.unpack_from("<I", p, 1)[0]
    ms = p[5]
    f = [struct.unpack_from("<H", p, 6 + 2 * i)[0] for i in range(ms + 1)]
    head = 6 + 2 * (ms + 1)
    head += (4 - head % 4) % 4
    nb = -(-n // BLOCK)
    off = [struct.unpack_from("<I", p, head + 4 * b)[0] for b in range(nb + 1)]
    data0 = head + 4 * (nb + 1)
    blocks = []
    for b in range(nb):
        blk = p[data0 + off[b]: data0 + off[b + 1]]
        nw = struct.unpack_from("<I", blk, 0)[0]
        states = struct.unpack_from("<64I", blk, 4)
        blocks.append((nw, states))
    return n, f, head, nb, off, data0, blocks


def test_hand_assembled_single_symbol_payload():
    # one symbol 5 with f[5] = 2048: lane 0 decodes it from state 2^16
    # (slot 0 -> symbol 5, x = 2048 * 32 + 0 = 2^16: no word), other lanes idle
    hdr = bytes([1]) + struct.pack("<I", 1) + bytes([5]) + struct.pack("<6H", 0, 0, 0, 0, 0, 2048)
    hdr += b"\0" * ((4 - len(hdr) % 4) % 4)
    block = struct.pack("<I", 0) + struct.pack("<64I", *([1 << 16] * 64))
    p = hdr + struct.pack("<II", 0, len(block)) + block
    assert O.rans_ilv_decode(p, 1) == b"\x05"
    bad = bytearray(p)
    struct.pack_into("<I", bad, len(hdr) + 8 + 4, (1 << 16) + 1)   # lane 0 does not end at 2^16
    with pytest.raises(O.OracleError):
        O.rans_ilv_decode(bytes(bad), 1)


def _cost_bound(plane, f):
    return sum(math.log2(2048 / f[s]) for s in plane)


@pytest.mark.parametrize("kind", ["geo", "nib", "skew", "bf16exp"])
def test_header_and_entropy_bound(kind):
    rng = np.random.default_rng(3)
    n = 3 * BLOCK + 1234
    if kind == "geo":
        x = rng.geometric(0.3, n).clip(0, 255).astype(np.uint8)
    elif kind == "nib":  # skewed nibbles (uniform ones are stored packed, see below)
        x = (16 - rng.geometric(0.3, n).clip(1, 16)).astype(np.uint8)
    elif kind == "skew":
        x = rng.choice([0, 1, 2, 200], n, p=[0.9, 0.05, 0.04, 0.01]).astype(np.uint8)
    else:
        x = np.clip(np.round(rng.normal(120, 1.5, n)), 0, 255).astype(np.uint8)
    p = O.rans_ilv_encode(x.tobytes())
    assert p[0] == 1
    n2, f, head, nb, off, data0, blocks = _parse(p)
    assert n2 == n and nb == 4 and off[0] == 0 and len(p) == data0 + off[-1]
    hist = np.bincount(x, minlength=256)
    want_f, _ = O.rans_normalize(hist)
    ms = int(np.nonzero(hist)[0].max())
    assert f == [int(v) for v in want_f[: ms + 1]]
    fa = [int(v) for v in want_f]
    for b, (nw, states) in enumerate(blocks):
        seg = x[b * BLOCK: (b + 1) * BLOCK]
        bits = _cost_bound(seg.tolist(), fa)
        # encoding a symbol of frequency f maps x to floor(x / f) 2048 + x mod f + cum,
        # i.e. x 2048 / f within a factor (1 +- f / x), x >= 32 f: so the state's
        # growth (16 bits per word plus the final states) is the symbols' cost
        # to within log2(33 / 32) bits per symbol
        growth = 16 * nw + sum(math.log2(s / 65536) for s in states)
        assert abs(growth - bits) <= len(seg) * math.log2(33 / 32) + 1e-6
        assert all((1 << 16) <= s < (1 << 32) for s in states)
    assert O.rans_ilv_decode(p, n) == x.tobytes()


def test_single_symbol_blocks_have_no_words():
    n = 2 * BLOCK + 7
    p = O.rans_ilv_encode(bytes([9]) * n)
    _, f, _, nb, off, _, blocks = _parse(p)
    assert f[9] == 2048 and nb == 3
    assert [b[0] for b in blocks] == [0, 0, 0] and off == [0, 260, 520, 780]
    assert O.rans_ilv_decode(p, n) == bytes([9]) * n


@pytest.mark.parametrize("n", [0, 1, 2, 15, 16, 17, 1023, 1024, 1025, BLOCK - 1, BLOCK, BLOCK + 1, 5 * BLOCK + 333])
def test_roundtrip_sizes(n):
    rng = np.random.default_rng(n)
    for x in (rng.geometric(0.2, n).clip(0, 255).astype(np.uint8), rng.integers(0, 256, n).astype(np.uint8),
              rng.integers(0, 3, n).astype(np.uint8)):
        p = O.rans_ilv_encode(x.tobytes())
        assert O.rans_ilv_decode(p, n) == x.tobytes()
        assert len(p) <= n + 1
        if p[0] == 0:
            assert p == b"\0" + x.tobytes()


def test_corruptions_rejected():
    rng = np.random.default_rng(11)
    x = rng.geometric(0.25, 2 * BLOCK + 100).clip(0, 255).astype(np.uint8).tobytes()
    p = O.rans_ilv_encode(x)
    n, f, head, nb, off, data0, blocks = _parse(p)
    rejected = 0
    for k in range(40):
        b = bytearray(p)
        i = int(rng.integers(data0 + 260, data0 + off[1]))  # a word byte of block 0
        b[i] ^= 1 << int(rng.integers(0, 8))
        try:
            rejected += O.rans_ilv_decode(bytes(b), n) != x
        except O.OracleError:
            rejected += 1
    assert rejected == 40
    b = bytearray(p)
    struct.pack_into("<I", b, data0, blocks[0][0] + 2)       # word count disagrees with the block size
    with pytest.raises(O.OracleError):
        O.rans_ilv_decode(bytes(b), n)
    with pytest.raises(O.OracleError):
        O.rans_ilv_decode(p[:-4], n)


@pytest.mark.parametrize("enc,dec", [(O.rans_ilv_encode, O.rans_ilv_decode), (O.ilv_encode, O.ilv_decode)],
                         ids=["rans_ilv", "huff_ilv"])
def test_packed_nibble_form(enc, dec):
    """Near-uniform nibble planes (MXFP4 codes) are stored two symbols per
    byte: [2][n u32][0 0 0][byte i = s[2i] | s[2i+1] << 4], the smallest of
    the three forms for them; malformed packed payloads are rejected."""
    rng = np.random.default_rng(4)
    for n in (16, 17, 18, 1001, 3 * BLOCK + 5):
        x = rng.integers(0, 16, n).astype(np.uint8)
        p = enc(x.tobytes())
        assert p[0] == 2 and struct.unpack_from("<I", p, 1)[0] == n and p[5:8] == b"\0\0\0"
        assert len(p) == 8 + (n + 1) // 2
        assert all(p[8 + i // 2] >> (4 * (i & 1)) & 15 == x[i] for i in range(n))
        assert dec(p, n) == x.tobytes()
    p = bytearray(enc(rng.integers(0, 16, 101).astype(np.uint8).tobytes()))
    for bad in (bytes(p[:-1]), bytes(p) + b"\0", bytes(p[:5]) + b"\1" + bytes(p[6:]),
                bytes(p[:-1]) + bytes([p[-1] | 0x10])):
        with pytest.raises(O.OracleError):
            dec(bad, 101)
    # a skewed nibble plane still codes (smaller than packed)
    y = (16 - rng.geometric(0.45, 20000).clip(1, 16)).astype(np.uint8)
    assert enc(y.tobytes())[0] == 1
