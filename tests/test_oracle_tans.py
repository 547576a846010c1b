"""tANS restatement (entropy/tans/mod.rs, codecs/tans.rs) pinned on CPU.

The golden pin is the reference's legacy fixtures: the chunked tensor
``model.layers.2.chunked.weight`` has a tANS plane of two chunk frames, and
its plane CRC-32 and the EXPECTED XXH64 of legacy_fixtures.rs:63-123 hold
after the oracle decodes it (test_container_cpu.py).  Here: the structural
invariants of the tables (a spread that fills every slot once, decode
next-state ranges that tile [0, L) per symbol -- what makes the coder
decodable at all), round trips, and the reference's rejections.
"""
import numpy as np
import pytest

L = 2048


def _norm(rng, nsym):
    """A normalized frequency table over nsym random symbols (sum L)."""
    syms = rng.choice(256, nsym, replace=False)
    cuts = np.sort(rng.choice(np.arange(1, L), nsym - 1, replace=False))
    f = np.diff(np.concatenate([[0], cuts, [L]]))
    norm = np.zeros(256, np.uint32)
    norm[syms] = f
    return norm


@pytest.mark.parametrize("nsym", [2, 3, 17, 256])
def test_spread_fills_every_slot_once_per_frequency(orc, nsym):
    norm = _norm(np.random.default_rng(nsym), nsym)
    table = orc.tans_spread(norm)
    counts = np.bincount(table, minlength=256)
    assert np.array_equal(counts, norm)
    # the first placement is slot 0 and the step is L/2 + L/8 + 3
    first = int(np.flatnonzero(norm)[0])
    assert table[0] == first
    assert table[1283] == (first if norm[first] > 1 else int(np.flatnonzero(norm)[1]))


@pytest.mark.parametrize("nsym", [2, 5, 64, 256])
def test_decode_ranges_tile_the_state_space(orc, nsym):
    norm = _norm(np.random.default_rng(100 + nsym), nsym)
    sym, nb, base = orc.tans_decode_table(norm)
    assert nb.max() <= 11
    for s in np.flatnonzero(norm):
        slots = np.flatnonzero(sym == s)
        ranges = sorted((int(base[u]), int(base[u]) + (1 << int(nb[u]))) for u in slots)
        assert ranges[0][0] == 0 and ranges[-1][1] == L
        for (a0, a1), (b0, b1) in zip(ranges, ranges[1:]):
            assert a1 == b0


def _samples():
    rng = np.random.default_rng(7)
    yield "two", np.array([3, 9] * 50, np.uint8)
    yield "geom", (rng.geometric(0.2, 5000) % 256).astype(np.uint8)
    yield "normal", np.clip(rng.normal(128, 6, 40000), 0, 255).astype(np.uint8)
    yield "uniform", rng.integers(0, 256, 3000, dtype=np.uint8)
    yield "runs", np.repeat(rng.integers(0, 4, 300), 17).astype(np.uint8)
    yield "skewed_full", np.concatenate([np.zeros(60000, np.uint8), np.arange(256, dtype=np.uint8)])


@pytest.mark.parametrize("name,data", list(_samples()))
def test_round_trip_and_framing(orc, name, data):
    blob = orc.tans_compress(data)
    if blob:
        assert blob[0] == 11
        assert orc.tans_decompress(blob, data.size) == data.tobytes()
    payload = orc.codec_encode(orc.CODEC_TANS, data)
    if blob:
        assert payload[0] == 1 and int.from_bytes(payload[1:5], "little") == data.size
        assert payload[5:] == blob
    else:
        assert payload == b"\x00" + data.tobytes()
    assert orc.codec_decode(orc.CODEC_TANS, payload, data.size) == data.tobytes()


def test_degenerate_inputs_store_raw(orc):
    assert orc.tans_compress(np.zeros(1000, np.uint8)) == b""
    assert orc.codec_encode(orc.CODEC_TANS, b"") == b"\x00"
    assert orc.codec_decode(orc.CODEC_TANS, b"\x00", 0) == b""
    assert orc.codec_encode(orc.CODEC_TANS, np.full(9, 4, np.uint8)) == b"\x00" + bytes([4] * 9)


def test_rejections(orc):
    rng = np.random.default_rng(3)
    data = (rng.geometric(0.3, 4000) % 256).astype(np.uint8)
    b = bytearray(orc.tans_compress(data))
    nsym = b[1] | (b[2] << 8)

    def rejects(blob, n=data.size):
        with pytest.raises(orc.OracleError):
            orc.tans_decompress(bytes(blob), n)

    bad = bytearray(b); bad[0] = 12; rejects(bad)                      # table_log
    bad = bytearray(b); bad[1:3] = (1).to_bytes(2, "little"); rejects(bad)    # nsym < 2
    bad = bytearray(b); bad[1:3] = (257).to_bytes(2, "little"); rejects(bad)  # nsym > 256
    bad = bytearray(b); bad[6] = bad[3]; rejects(bad)                  # duplicate symbol
    bad = bytearray(b); bad[4:6] = b"\x00\x00"; rejects(bad)           # zero frequency
    bad = bytearray(b); bad[4] ^= 1; rejects(bad)                      # sum != L
    tb = 3 + 3 * nsym
    bits = int.from_bytes(b[tb:tb + 8], "little")
    bad = bytearray(b); bad[tb:tb + 8] = (8 * (len(b) - tb - 8) + 1).to_bytes(8, "little"); rejects(bad)
    bad = bytearray(b); bad[tb:tb + 8] = (bits + 1).to_bytes(8, "little"); rejects(bad)  # trailing bits
    rejects(b[:tb + 4])                                                # truncated header
    rejects(b, data.size + 1)                                          # one symbol too many
    rejects(b, data.size - 1)                                          # stream not consumed
    rejects(b[:2])
    # payload framing (codecs/tans.rs:101-137)
    with pytest.raises(orc.OracleError):
        orc.codec_decode(orc.CODEC_TANS, b"", 10)                      # empty payload
    with pytest.raises(orc.OracleError):
        orc.codec_decode(orc.CODEC_TANS, b"\x02abc", 10)               # bad tag
    with pytest.raises(orc.OracleError):
        orc.codec_decode(orc.CODEC_TANS, b"\x01\x05\x00", 10)          # short prefix
    p = b"\x01" + data.size.to_bytes(4, "little") + bytes(b)
    with pytest.raises(orc.OracleError):
        orc.codec_decode(orc.CODEC_TANS, p, data.size - 1)             # declared > bound
    assert orc.codec_decode(orc.CODEC_TANS, p, data.size) == data.tobytes()
