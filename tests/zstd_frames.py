"""Zstandard frames written by the image's libzstd (test helper, not a test).

The reference's Zstd plane codec writes its payloads with libzstd
(zstd crate 0.13.3, codecs/zstd.rs: level 3, encode_all).  The image ships
libzstd.so.1; frames made here with its advanced parameters (level, window,
checksum, content size) cover the block and table forms the oracle's
RFC 8878 restatement and the device decoder must read.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

_z = None
ZSTD_c_compressionLevel = 100
ZSTD_c_windowLog = 101
ZSTD_c_contentSizeFlag = 200
ZSTD_c_checksumFlag = 201


def lib():
    global _z
    if _z is None:
        z = C.CDLL("libzstd.so.1")
        z.ZSTD_createCCtx.restype = C.c_void_p
        z.ZSTD_freeCCtx.argtypes = [C.c_void_p]
        z.ZSTD_CCtx_setParameter.argtypes = [C.c_void_p, C.c_int, C.c_int]
        z.ZSTD_CCtx_setParameter.restype = C.c_size_t
        z.ZSTD_compress2.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t]
        z.ZSTD_compress2.restype = C.c_size_t
        z.ZSTD_compressBound.argtypes = [C.c_size_t]
        z.ZSTD_compressBound.restype = C.c_size_t
        z.ZSTD_isError.argtypes = [C.c_size_t]
        z.ZSTD_isError.restype = C.c_uint
        _z = z
    return _z


def compress(data: bytes, level: int = 3, checksum: bool = False, content_size: bool = True,
             window_log: int = 0) -> bytes:
    z = lib()
    cc = z.ZSTD_createCCtx()
    try:
        for p, v in ((ZSTD_c_compressionLevel, level), (ZSTD_c_checksumFlag, int(checksum)),
                     (ZSTD_c_contentSizeFlag, int(content_size))):
            assert not z.ZSTD_isError(z.ZSTD_CCtx_setParameter(cc, p, v))
        if window_log:
            assert not z.ZSTD_isError(z.ZSTD_CCtx_setParameter(cc, ZSTD_c_windowLog, window_log))
        cap = z.ZSTD_compressBound(len(data))
        out = C.create_string_buffer(cap)
        n = z.ZSTD_compress2(cc, out, cap, data, len(data))
        assert not z.ZSTD_isError(n)
        return out.raw[:n]
    finally:
        z.ZSTD_freeCCtx(cc)


def skippable(payload: bytes, k: int = 0) -> bytes:
    return (0x184D2A50 + k).to_bytes(4, "little") + len(payload).to_bytes(4, "little") + payload


def samples(seed: int = 0):
    """Plane-like byte strings of several statistics (name, bytes)."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal(150_000) * 0.02).astype(np.float32)
    hi = (w.view(np.uint32) >> 24).astype(np.uint8)   # exponent-like plane
    yield "exp-plane", hi.tobytes()
    yield "bf16-high", (((w.view(np.uint32) >> 16) & 0xFF).astype(np.uint8)).tobytes()
    yield "geom", (rng.geometric(0.15, 300_000) % 256).astype(np.uint8).tobytes()
    yield "text", b"".join(b"tensor %d has %d planes; " % (i, i % 7) for i in range(9000))
    yield "zeros", bytes(200_000)
    yield "random", rng.integers(0, 256, 70_000, dtype=np.uint8).tobytes()
    yield "runs", np.repeat(rng.integers(0, 6, 4000), rng.integers(1, 90, 4000)).astype(np.uint8).tobytes()
    yield "tiny", b"ab"
    yield "empty", b""
