"""Trial-encode selection (select.rs:27-64, dispatch.rs:13-49) in the oracle.

Pins: the reference's own known answers (select.rs tests: Identity wins on a
1 KiB high-entropy plane, Huffman on 4 KiB of zeros, an empty menu is an
error); the tie rule (min_by_key keeps the first of equal sizes); and that
the winner's payload is exactly the smallest of the menu's encodes.
"""
import numpy as np
import pytest


def test_reference_known_answers(orc):
    hi = np.array([((i * 12347) ^ 0x5A5A5A5A) & 0xFF for i in range(1024)], np.uint8)
    assert orc.select_encode(hi, (orc.CODEC_IDENTITY, orc.CODEC_HUFFMAN))[0] == orc.CODEC_IDENTITY
    z = np.zeros(4096, np.uint8)
    assert orc.select_encode(z, (orc.CODEC_IDENTITY, orc.CODEC_HUFFMAN))[0] == orc.CODEC_HUFFMAN
    with pytest.raises(orc.OracleError):
        orc.select_encode(z, ())


def test_ties_go_to_the_first_in_menu(orc):
    # incompressible: Huffman and rANS both store raw (n + 1 bytes)
    x = np.random.default_rng(0).integers(0, 256, 5000, dtype=np.uint8)
    h = orc.codec_encode(orc.CODEC_HUFFMAN, x)
    r = orc.codec_encode(orc.CODEC_RANS, x)
    assert len(h) == len(r) == x.size + 1
    assert orc.select_encode(x, (orc.CODEC_HUFFMAN, orc.CODEC_RANS))[0] == orc.CODEC_HUFFMAN
    assert orc.select_encode(x, (orc.CODEC_RANS, orc.CODEC_HUFFMAN))[0] == orc.CODEC_RANS
    assert orc.select_encode(x)[0] == orc.CODEC_IDENTITY  # the default menu: Identity (n bytes) wins


@pytest.mark.parametrize("seed", range(6))
def test_winner_is_the_smallest_encode(orc, seed):
    rng = np.random.default_rng(seed)
    kind = seed % 3
    if kind == 0:
        x = rng.geometric(0.3, 20000).clip(0, 255).astype(np.uint8)
    elif kind == 1:
        x = np.clip(rng.normal(128, 20, 30000), 0, 255).astype(np.uint8)
    else:
        x = rng.integers(0, 4, 10000).astype(np.uint8)
    codec, payload = orc.select_encode(x)
    sizes = [len(orc.codec_encode(c, x)) for c in orc.DEFAULT_MENU]
    assert len(payload) == min(sizes)
    assert orc.DEFAULT_MENU.index(codec) == sizes.index(min(sizes))
    assert payload == orc.codec_encode(codec, x)
    assert orc.codec_decode(codec, payload, x.size) == x.tobytes()
