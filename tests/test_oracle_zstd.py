"""Zstd restatement (oracle/zstd_oracle.c, RFC 8878) pinned on CPU.

Pins: the reference's own Zstd planes (every Zstd plane of the golden legacy
fixtures and PTWS frames decodes to the bytes whose CRC-32 and XXH64 the
files hold: test_container_cpu.py), and frames written by the image's
libzstd at every level, with and without checksum / content size, several
windows, concatenated and with skippable frames; malformed frames are
rejected as libzstd's decoder rejects them.
"""
import numpy as np
import pytest

import zstd_frames as ZF

SAMPLES = list(ZF.samples())
LEVELS = [-5, 1, 3, 9, 19]


@pytest.mark.parametrize("name,data", SAMPLES, ids=[n for n, _ in SAMPLES])
@pytest.mark.parametrize("level", LEVELS)
def test_libzstd_frames_decode(orc, name, data, level):
    f = ZF.compress(data, level)
    assert orc.zstd_decompress(f, len(data)) == data
    assert orc.codec_decode(orc.CODEC_ZSTD, f, len(data)) == data


@pytest.mark.parametrize("name,data", SAMPLES[:4], ids=[n for n, _ in SAMPLES[:4]])
def test_frame_options(orc, name, data):
    for kw in (dict(checksum=True), dict(content_size=False), dict(window_log=10), dict(window_log=17, level=19),
               dict(checksum=True, content_size=False, level=1)):
        f = ZF.compress(data, **kw)
        assert orc.zstd_decompress(f, len(data)) == data, kw


def test_concatenated_and_skippable_frames(orc):
    a, b = SAMPLES[0][1][:50_000], SAMPLES[2][1][:70_000]
    blob = ZF.skippable(b"meta") + ZF.compress(a, 3) + ZF.skippable(b"", 5) + ZF.compress(b, 1, checksum=True)
    assert orc.zstd_decompress(blob, len(a) + len(b)) == a + b
    assert orc.zstd_decompress(b"", 10) == b""


def test_rejections(orc):
    data = SAMPLES[2][1][:100_000]
    f = bytearray(ZF.compress(data, 3, checksum=True))

    def rejects(blob, cap=len(data)):
        with pytest.raises(orc.OracleError):
            orc.zstd_decompress(bytes(blob), cap)

    rejects(f, len(data) - 1)                         # bound: zstd_read_bounded
    rejects(f[:-1])                                   # truncated checksum
    bad = bytearray(f); bad[-1] ^= 0xFF; rejects(bad)  # checksum mismatch
    bad = bytearray(f); bad[0] ^= 1; rejects(bad)     # magic
    bad = bytearray(f); bad[4] |= 0x08; rejects(bad)  # reserved bit
    rejects(f + b"\x00")                              # trailing garbage (not a frame)
    rejects(f[: len(f) // 2])                         # truncated block
    # a dictionary id: the plane codec has no dictionary
    d = bytearray(ZF.compress(b"abcdef" * 100, 3))
    fhd = d[4]
    withdict = d[:4] + bytes([fhd | 1]) + d[5:6 if not (fhd & 0x20) else 5] + b"\x07" + d[(6 if not (fhd & 0x20) else 5):]
    rejects(withdict)


def test_corrupt_block_bytes_never_overrun(orc):
    """Random corruption of a compressed frame: the restatement either
    rejects it or returns at most `cap` bytes (it runs in-process)."""
    data = SAMPLES[0][1][:60_000]
    f = ZF.compress(data, 3)
    rng = np.random.default_rng(1)
    for _ in range(400):
        b = bytearray(f)
        for pos in rng.integers(6, len(b), 3):
            b[pos] ^= int(rng.integers(1, 256))
        try:
            out = orc.zstd_decompress(bytes(b), len(data))
            assert len(out) <= len(data)
        except orc.OracleError:
            pass
