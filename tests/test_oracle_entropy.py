"""Oracle checks: Huffman, rANS, stream frame, plane payloads, chunk framing.

What pins each function (no reference code can run here: no Rust toolchain):
- reference unit-test known answers (cited per test);
- hand-derived vectors built from the wire format (bit order, jump table,
  weight header, rANS state update from the textbook rANS definition);
- mathematical properties: Huffman cost optimality against an independent
  textbook Huffman on small alphabets, Kraft sums, canonical ordering,
  reciprocal == div/mod for every (state, freq) class, round trips;
- decoder error paths the reference tests exercise.
"""
import heapq

import numpy as np
import pytest

import oracle as O


def rb(seed, n, hi=256):
    return np.random.default_rng(seed).integers(0, hi, n, dtype=np.uint8).tobytes()


# ---------------- stream frame (entropy/stream_frame.rs:64-116) -------------

def test_split_four_known_answers(orc):
    import ctypes as C
    s = (C.c_size_t * 4)(); e = (C.c_size_t * 4)()
    orc.lib().por_split_four(11, s, e)
    assert list(zip(s, e)) == [(0, 3), (3, 6), (6, 9), (9, 11)]
    orc.lib().por_split_four(16, s, e)
    assert (s[0], e[0], s[3], e[3]) == (0, 4, 12, 16)
    orc.lib().por_split_four(0, s, e)
    assert list(e) == [0, 0, 0, 0]


# ---------------- weights header (entropy/huffman/weights.rs:87-173) ---------

def test_weights_header_bytes(orc):
    w127 = bytes((i % 11) + 1 for i in range(127))
    enc = O.huf_encode_weights(w127)
    assert enc[0] == 0x80 | 127
    assert O.huf_decode_weights(enc) == (w127, len(enc))
    w128 = bytes((i % 11) + 1 for i in range(128))
    enc = O.huf_encode_weights(w128)
    assert enc[:2] == bytes([0x80, 128])
    assert O.huf_decode_weights(enc) == (w128, len(enc))
    w256 = bytes((i % 11) + 1 for i in range(256))
    enc = O.huf_encode_weights(w256)
    assert enc[:2] == bytes([0x80, 0])
    assert O.huf_decode_weights(enc) == (w256, len(enc))
    enc = O.huf_encode_weights(bytes([3, 5, 7]))
    assert enc == bytes([0x83, 0x53, 0x07])           # low nibble first, odd count padded


def test_weights_decode_rejects(orc):
    for bad in (b"\x42", b"\x80", b"", b"\x80\x05", b"\x85\x11"):
        with pytest.raises(O.OracleError):
            O.huf_decode_weights(bad)
    with pytest.raises(O.OracleError):
        O.huf_encode_weights(b"")
    with pytest.raises(O.OracleError):
        O.huf_encode_weights(bytes(257))


# ---------------- tree (entropy/huffman/tree.rs:253-348) ---------------------

def freqs_of(d):
    f = np.zeros(256, np.uint32)
    for k, v in d.items():
        f[k] = v
    return f


def test_tree_single_and_two_symbols(orc):
    L = O.huf_lengths(freqs_of({42: 1000}))
    assert L[42] == 1 and L.sum() == 1
    mb, table, _ = O.huf_table(L)
    assert mb == 1 and len(table) == 2
    L = O.huf_lengths(freqs_of({0: 100, 255: 50}))
    assert L[0] == 1 and L[255] == 1
    mb, table, _ = O.huf_table(L)
    assert mb == 1 and len(table) == 2
    assert O.huf_lengths(np.zeros(256, np.uint32)) is None
    assert O.huf_table(np.array([12] + [0] * 255)) is None


def test_tree_skewed_is_length_limited(orc):
    f = np.ones(256, np.uint32)
    f[0] = 1 << 20
    L = O.huf_lengths(f)
    assert L.max() <= 11 and 0 < L[0] < L[1]
    assert sum(2.0 ** -int(l) for l in L if l) <= 1.0


def textbook_huffman_cost(freqs):
    """Independent textbook Huffman: optimal total bits for a prefix code."""
    h = [f for f in freqs if f > 0]
    if len(h) == 1:
        return h[0]
    heapq.heapify(h)
    cost = 0
    while len(h) > 1:
        a = heapq.heappop(h); b = heapq.heappop(h)
        cost += a + b
        heapq.heappush(h, a + b)
    return cost


@pytest.mark.parametrize("seed", range(40))
def test_tree_optimal_and_canonical(orc, seed):
    rng = np.random.default_rng(seed)
    k = int(rng.integers(2, 40))
    syms = rng.choice(256, k, replace=False)
    f = np.zeros(256, np.uint32)
    f[syms] = rng.integers(1, 1000, k)
    L = O.huf_lengths(f)
    # optimal unless the 11-bit limit had to kick in
    if L.max() < 11:
        assert int((L.astype(np.int64) * f).sum()) == textbook_huffman_cost([int(x) for x in f])
        assert sum(2.0 ** -int(l) for l in L if l) == 1.0     # complete tree
    mb, table, rev = O.huf_table(L)
    # canonical: codes increase with (length, symbol); decode table inverts them
    codes = []
    for s in range(256):
        if L[s]:
            code = int("".join(str((int(rev[s]) >> i) & 1) for i in range(L[s])), 2)
            codes.append((int(L[s]), s, code))
    codes.sort()
    prev_len, prev_code = 0, -1
    for l, s, c in codes:
        nxt = (prev_code + 1) << (l - prev_len) if prev_len else 0
        assert c == nxt
        prev_len, prev_code = l, c
        for i in range(1 << (mb - l)):
            assert table[int(rev[s]) | (i << l)] == (l << 8) | s


def test_tree_tie_break_is_by_symbol_order(orc):
    """Equal frequencies: leaves pop in ascending symbol id (tree.rs:51-65)."""
    L = O.huf_lengths(freqs_of({1: 5, 2: 5, 3: 5}))
    # ids 0(sym1),1(sym2) merge first -> sym3 gets the 1-bit code
    assert (L[1], L[2], L[3]) == (2, 2, 1)
    L = O.huf_lengths(freqs_of({10: 3, 20: 3, 30: 6}))
    assert (L[10], L[20], L[30]) == (2, 2, 1)
    L = O.huf_lengths(freqs_of({10: 1, 20: 1, 30: 1, 40: 1, 50: 4}))
    assert list(L[[10, 20, 30, 40, 50]]) == [3, 3, 3, 3, 1]


def test_tree_weights_roundtrip(orc):
    L = O.huf_lengths(freqs_of({0: 500, 1: 200, 2: 100, 3: 50, 4: 10}))
    n = max(i for i in range(256) if L[i]) + 1
    w, _ = O.huf_decode_weights(O.huf_encode_weights(L[:n].tobytes()))
    assert np.array_equal(np.frombuffer(w, np.uint8), L[:n])


# ---------------- backward bitstream (bitstream.rs:189-234) ------------------

def test_bitstream_layout(orc):
    # bits are consumed LSB-first from the LAST byte backwards
    s = O.bitwriter_pack([(0b01, 2), (0b101, 3), (0b1111, 4)])
    # forward bit string: 1,0 | 1,0,1 | 1,1,1,1  -> k=0..8
    bits = [1, 0, 1, 0, 1, 1, 1, 1, 1]
    m = (len(bits) + 7) // 8
    assert len(s) == m
    for k, b in enumerate(bits):
        assert (s[m - 1 - k // 8] >> (k % 8)) & 1 == b
    assert s[0] >> 1 == 0                          # zero padding
    codes = [((i * 3 + 1) & 0x7FF, 11) for i in range(50)]
    s = O.bitwriter_pack(codes)
    assert len(s) == (50 * 11 + 7) // 8
    k = 0
    for c, n in codes:
        for i in range(n):
            assert (s[len(s) - 1 - k // 8] >> (k % 8)) & 1 == (c >> i) & 1
            k += 1


# ---------------- Huffman compress/decompress (huffman/mod.rs:45-299) --------

def test_huffman_hand_derived_vector(orc):
    """48 x 0 then 16 x 1 style segments: 2 symbols, both 1-bit codes
    (sym0 -> 0, sym1 -> 1), weights header 0x82 0x11."""
    seg0 = [0] * 16
    seg1 = [0, 1, 0, 0, 0, 0, 0, 0, 1, 1, 1, 1, 0, 0, 0, 0]
    seg2 = [0] * 16
    seg3 = [1] * 16
    src = bytes(seg0 + seg1 + seg2 + seg3)
    oc, blob = O.huf_compress(src)
    assert oc == O.OUT_ENCODED
    expect = bytes([0x82, 0x11]) + bytes([2, 0, 0, 0] * 4) + bytes([0, 0, 0x0F, 0x02, 0, 0, 0xFF, 0xFF])
    assert blob == expect
    assert O.huf_decompress(blob, len(src)) == src


@pytest.mark.parametrize("src", [
    bytes(i % 64 for i in range(4096)),
    bytes([0] * 3000 + [200] * 600 + [128] * 200 + [255] * 100),
    bytes([42] * 1024),
    bytes([0] * 3000 + [1] * 1000),
    bytes(i % 32 for i in range(65536)),
    bytes(i % 50 for i in range(4093)),
])
def test_huffman_roundtrip_reference_cases(orc, src):
    oc, blob = O.huf_compress(src)
    assert oc == O.OUT_ENCODED and 0 < len(blob) < len(src)
    assert O.huf_decompress(blob, len(src)) == src


def test_huffman_not_encoded_cases(orc):
    assert O.huf_compress(bytes((i * 137 + 42) & 0xFF for i in range(32)))[0] != O.OUT_ENCODED
    assert O.huf_compress(bytes(b for b in range(256)) * 4)[0] != O.OUT_ENCODED
    assert O.huf_compress(b"")[0] == O.OUT_INCOMPRESSIBLE
    oc, _ = O.huf_compress(bytes(100), cap=10)
    assert oc == O.OUT_DST_TOO_SMALL                 # compress.rs:118-126


def test_huffman_2mb_low_entropy(orc):
    i = np.arange(2 * 1024 * 1024)
    src = np.where(i % 10 == 0, (i >> 3) & 0x0F, 0).astype(np.uint8).tobytes()
    oc, blob = O.huf_compress(src)
    assert oc == O.OUT_ENCODED and len(blob) < len(src) // 2
    assert O.huf_decompress(blob, len(src)) == src


def test_huffman_decoder_errors(orc):
    with pytest.raises(O.OracleError):
        O.huf_decompress(b"\x80", 64)
    with pytest.raises(O.OracleError):
        O.huf_decompress(bytes([0x82, 0x11, 0, 0, 0]), 64)       # truncated jump table
    with pytest.raises(O.OracleError):
        O.huf_decompress(b"", 64)
    with pytest.raises(O.OracleError):
        O.huf_decompress(bytes([0xFF, 0, 0, 0]), 64)
    src = bytes(i % 64 for i in range(4096))
    _, blob = O.huf_compress(src)
    with pytest.raises(O.OracleError):
        O.huf_decompress(blob[: len(blob) // 2], len(src))
    bad = bytearray(blob)
    bad[len(bad) // 2] ^= 0xFF
    bad[len(bad) // 2 + 1] ^= 0xFF
    try:
        assert O.huf_decompress(bytes(bad), len(src)) != src
    except O.OracleError:
        pass
    for seed in range(16):                                      # garbage never crashes
        g = bytes(((i * (seed + 17)) * 31) & 0xFF for i in range(2048))
        try:
            O.huf_decompress(g, 1024)
        except O.OracleError:
            pass


def test_huffman_trailing_garbage_bits_rejected(orc):
    """A set padding bit leaves the reader's container non-zero (is_exhausted)."""
    src = bytes([0] * 3 + [1]) * 16
    _, blob = O.huf_compress(src)
    bad = bytearray(blob)
    # stream 0 = segment [0,0,0,1]*4: 16 bits -> 2 bytes, no padding; extend it
    O.huf_decompress(blob, len(src))
    # a stream with an extra leading zero byte is still all-loaded and zero: accepted
    jt = 2
    lens = [int.from_bytes(bad[jt + 4 * i: jt + 4 * i + 4], "little") for i in range(4)]
    body = bytes(bad[jt + 16:])
    s0 = body[: lens[0]]
    alt = bytes(bad[:jt]) + (lens[0] + 1).to_bytes(4, "little") + bytes(bad[jt + 4: jt + 16]) + b"\x00" + body
    assert O.huf_decompress(alt, len(src)) == src
    alt2 = bytes(bad[:jt]) + (lens[0] + 1).to_bytes(4, "little") + bytes(bad[jt + 4: jt + 16]) + b"\x01" + body
    with pytest.raises(O.OracleError):
        O.huf_decompress(alt2, len(src))
    del s0


# ---------------- rANS (entropy/rans/{compress,decompress,mod}.rs) -----------

def test_rans_normalize_known_answers(orc):
    f, cum = O.rans_normalize(freqs_of({0: 3000, 1: 1000}))
    assert int(f.sum()) == 2048 and cum[0] == 0 and cum[1] == f[0]
    assert (f[0], f[1]) == (1536, 512)
    assert O.rans_normalize(np.zeros(256, np.uint32)) is None
    # excess absorbed by the FIRST most frequent symbol
    raw = np.zeros(256, np.uint32)
    raw[:256] = 1
    raw[7] = 10
    raw[9] = 10
    f, _ = O.rans_normalize(raw)
    assert int(f.sum()) == 2048 and f[7] != f[9]


def test_rans_reciprocal_equals_divmod(orc):
    """compress.rs:164-176: the reciprocal update equals (x/f)*M + x%f + start."""
    L = orc.lib()
    rng = np.random.default_rng(5)
    for freq in list(range(1, 40)) + [511, 512, 513, 1000, 1023, 1024, 1025, 2047, 2048]:
        start = 0 if freq == 2048 else int(rng.integers(0, 2048 - freq + 1))
        hi = (1 << 20) * freq
        for x in [1, hi - 1, 1 << 15, (1 << 23) + 1] + [int(v) for v in rng.integers(1, hi, 200)]:
            if x >= hi:
                continue
            assert L.por_rans_enc_update(x, start, freq) == (x // freq) * 2048 + x % freq + start


def textbook_rans_encode_segment(seg, f, cum):
    x = 1 << 23
    out = []
    for s in reversed(seg):
        fs = int(f[s])
        while x >= ((1 << 23) >> 11 << 8) * fs:
            out.append(x & 0xFF)
            x >>= 8
        x = (x // fs) * 2048 + (x % fs) + int(cum[s])
    return x.to_bytes(4, "little") + bytes(reversed(out))


def test_rans_hand_derived_vector(orc):
    src = bytes([0, 0, 0, 1] * 16)
    oc, blob = O.rans_compress(src)
    assert oc == O.OUT_ENCODED
    f = np.zeros(256, np.uint32); f[0] = 1536; f[1] = 512
    cum = np.zeros(256, np.uint32); cum[1] = 1536
    streams = [textbook_rans_encode_segment(src[16 * i:16 * i + 16], f, cum) for i in range(4)]
    expect = bytes([1, 0x00, 0x06, 0x00, 0x02]) + b"".join(len(s).to_bytes(4, "little") for s in streams) + b"".join(streams)
    assert blob == expect
    assert O.rans_decompress(blob, len(src)) == src


@pytest.mark.parametrize("k", range(12))
def test_rans_roundtrip_diverse(orc, k):
    rng = np.random.default_rng(100 + k)
    n = int(rng.integers(1, 20000))
    alpha = int(rng.integers(1, 257))
    p = rng.dirichlet(np.ones(alpha) * (0.05 + k * 0.3))
    src = rng.choice(alpha, n, p=p).astype(np.uint8).tobytes()
    oc, blob = O.rans_compress(src)
    if oc == O.OUT_ENCODED:
        assert O.rans_decompress(blob, n) == src


def test_rans_not_encoded_and_errors(orc):
    assert O.rans_compress(bytes(range(256)) * 4)[0] != O.OUT_ENCODED
    assert O.rans_compress(b"")[0] == O.OUT_INCOMPRESSIBLE
    with pytest.raises(O.OracleError):
        O.rans_decompress(b"", 10)
    with pytest.raises(O.OracleError):
        O.rans_decompress(bytes([1, 0, 4, 0, 4]), 10)       # sum != 2048
    _, blob = O.rans_compress(bytes([0, 0, 0, 1] * 256))
    with pytest.raises(O.OracleError):
        O.rans_decompress(blob[:-3], 1024)                   # jump table sum mismatch


# ---------------- plane payloads (codecs/*.rs) -------------------------------

@pytest.mark.parametrize("codec", [O.CODEC_HUFFMAN, O.CODEC_RANS])
def test_codec_payload_framing(orc, codec):
    assert O.codec_encode(codec, b"") == b"\x00"
    raw = rb(3, 1000)
    assert O.codec_encode(codec, raw) == b"\x00" + raw            # not beneficial -> raw
    src = bytes(i % 16 for i in range(5000))
    p = O.codec_encode(codec, src)
    assert p[0] == 1 and int.from_bytes(p[1:5], "little") == 5000
    assert O.codec_decode(codec, p, 5000) == src
    assert O.codec_decode(codec, b"\x00abc", 3) == b"abc"
    for bad in (b"", b"\x02", b"\x01\x00\x00"):
        with pytest.raises(O.OracleError):
            O.codec_decode(codec, bad, 10)


def test_huffman_orig_len_cap(orc):
    # codecs/huffman.rs:122-131: orig_len <= 32 * encoded + 4096
    with pytest.raises(O.OracleError):
        O.codec_decode(O.CODEC_HUFFMAN, b"\x01" + (5000).to_bytes(4, "little") + b"\x82\x11", 10**6)


def test_rans_orig_len_zero_is_empty(orc):
    # codec_tagged.rs:108-110: expected_len == 0 returns empty without decoding
    assert O.codec_decode(O.CODEC_RANS, b"\x01\x00\x00\x00\x00garbage", 0) == b""


def test_identity_payload(orc):
    assert O.codec_encode(O.CODEC_IDENTITY, b"xyz") == b"xyz"
    assert O.codec_decode(O.CODEC_IDENTITY, b"xyz", 3) == b"xyz"


# ---------------- chunk framing (compressor.rs:316-381) ----------------------

@pytest.mark.parametrize("codec", [O.CODEC_IDENTITY, O.CODEC_HUFFMAN, O.CODEC_RANS])
def test_chunked_roundtrip_and_layout(orc, codec):
    src = bytes(np.random.default_rng(1).geometric(0.3, 70000).clip(0, 255).astype(np.uint8))
    payload, ent = O.encode_plane_chunked(codec, src, 16384)
    assert ent.shape[0] == 5 and ent[0, 0] == 0 and list(ent[:, 1]) == [16384] * 4 + [70000 - 4 * 16384]
    for k in range(5):
        o = int(ent[k, 0])
        assert payload[o:o + 5] == b"\x00\x00\x00\x00\x00"
        end = int(ent[k + 1, 0]) if k < 4 else len(payload)
        assert O.codec_decode(codec, payload[o + 5:end], 16384) == src[16384 * k:16384 * k + int(ent[k, 1])]
    assert O.decode_plane_chunked(codec, payload, ent) == src
    assert O.decode_plane_chunked(codec, payload, ent, threads=4) == src


def test_chunked_empty_plane(orc):
    payload, ent = O.encode_plane_chunked(O.CODEC_HUFFMAN, b"", 1024)
    assert payload == b"\x00\x00\x00\x00\x00\x00" and ent.tolist() == [[0, 0]]
