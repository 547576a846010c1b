"""ctypes view of the CPU oracle (``oracle/_build/libptwm_oracle.so``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg, always as the checker or the timed
CPU baseline, never as the product path.  The C sources restate the
reference algorithms (``crates/ptwm-core/src/...``); each C function cites
the reference file:line it follows.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libptwm_oracle.so")

CODEC_IDENTITY = 0x0000
CODEC_HUFFMAN = 0x0001
CODEC_RANS = 0x0003
CODEC_ZSTD = 0x0004
CODEC_TANS = 0x0007

CHAIN_IEEE16_SPLIT2 = 1
CHAIN_IEEE32_SPLIT4 = 2
CHAIN_E4M3_NIBBLE = 3
CHAIN_E5M2_NIBBLE = 4
CHAIN_NIBBLE_SPLIT = 5
CHAIN_PASSTHROUGH = 6

OUT_ENCODED, OUT_NOT_BENEFICIAL, OUT_INCOMPRESSIBLE, OUT_DST_TOO_SMALL, OUT_LEN_OVERFLOW = range(5)


class OracleError(RuntimeError):
    """A negative return code from the oracle (the reference returned Err)."""

    def __init__(self, rc: int, what: str):
        super().__init__(f"{what}: rc={rc}")
        self.rc = rc


def build() -> str:
    """Compile the oracle with gcc (oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


_lib = None
u8p = C.POINTER(C.c_uint8)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        sz, i64, vp = C.c_size_t, C.c_int64, C.c_void_p
        L.por_huf_compress.restype = i64
        L.por_huf_compress.argtypes = [vp, sz, vp, sz, C.POINTER(C.c_int)]
        L.por_huf_decompress.restype = i64
        L.por_huf_decompress.argtypes = [vp, sz, vp, sz]
        L.por_rans_compress.restype = i64
        L.por_rans_compress.argtypes = [vp, sz, vp, sz, C.POINTER(C.c_int)]
        L.por_rans_decompress.restype = i64
        L.por_rans_decompress.argtypes = [vp, sz, vp, sz]
        L.por_codec_encode.restype = i64
        L.por_zstd_decompress.argtypes = [vp, sz, vp, sz]
        L.por_zstd_decompress.restype = C.c_int64
        L.por_select_encode.argtypes = [vp, sz, vp, sz, vp, vp, sz]
        L.por_select_encode.restype = C.c_int64
        L.por_tans_compress.argtypes = [vp, sz, vp, sz]
        L.por_tans_compress.restype = C.c_int64
        L.por_tans_decompress.argtypes = [vp, sz, vp, sz]
        L.por_tans_decompress.restype = C.c_int64
        L.por_tans_decode_table.argtypes = [vp, vp, vp, vp]
        L.por_tans_spread.argtypes = [vp, vp]
        L.por_codec_encode.argtypes = [C.c_int, vp, sz, vp, sz]
        L.por_codec_decode.restype = i64
        L.por_codec_decode.argtypes = [C.c_int, vp, sz, vp, sz]
        L.por_codec_decoded_len.restype = i64
        L.por_codec_decoded_len.argtypes = [C.c_int, vp, sz]
        L.por_codec_encode_bound.restype = sz
        L.por_codec_encode_bound.argtypes = [sz]
        L.por_encode_plane_chunked.restype = i64
        L.por_encode_plane_chunked.argtypes = [C.c_int, vp, sz, C.c_uint32, vp, sz, vp, sz, C.POINTER(sz)]
        L.por_decode_plane_chunked.restype = i64
        L.por_decode_plane_chunked.argtypes = [C.c_int, vp, sz, vp, sz, vp, sz]
        L.por_decode_plane_chunked_mt.restype = i64
        L.por_decode_plane_chunked_mt.argtypes = [C.c_int, vp, sz, vp, sz, vp, sz, C.c_int]
        L.por_decode_tensors_mt.restype = i64
        L.por_decode_tensors_mt.argtypes = [C.c_int, C.c_int, sz, vp, vp, vp, vp, vp, vp, C.c_int]
        L.por_batch_decode_mt.restype = i64
        L.por_batch_decode_mt.argtypes = [sz, vp, vp, vp, vp, vp, vp, vp, vp, vp, C.c_int]
        L.por_batch_encode_mt.restype = i64
        L.por_batch_encode_mt.argtypes = [sz, vp, vp, vp, vp, vp, vp, vp, vp, vp, C.c_int]
        L.por_huf_lengths_from_freqs.restype = C.c_int
        L.por_huf_lengths_from_freqs.argtypes = [vp, vp]
        L.por_huf_lengths_limited.restype = C.c_int
        L.por_huf_lengths_limited.argtypes = [vp, vp, C.c_int]
        L.por_ilv_lengths.restype = C.c_int
        L.por_ilv_lengths.argtypes = [vp, vp]
        L.por_huf_from_lengths.restype = C.c_int
        L.por_huf_from_lengths.argtypes = [vp, vp, vp]
        L.por_huf_encode_weights.restype = i64
        L.por_huf_encode_weights.argtypes = [vp, sz, vp, sz]
        L.por_huf_decode_weights.restype = i64
        L.por_huf_decode_weights.argtypes = [vp, sz, vp, C.POINTER(C.c_int)]
        L.por_bitwriter_pack.restype = i64
        L.por_bitwriter_pack.argtypes = [vp, vp, sz, vp, sz]
        L.por_rans_normalize.restype = C.c_int
        L.por_rans_normalize.argtypes = [vp, vp, vp]
        L.por_rans_enc_update.restype = C.c_uint32
        L.por_rans_enc_update.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32]
        L.por_chain_forward.restype = C.c_int
        L.por_chain_forward.argtypes = [C.c_int, vp, sz, vp]
        L.por_chain_inverse.restype = C.c_int
        L.por_chain_inverse.argtypes = [C.c_int, vp, sz, vp]
        L.por_chain_plane_len.restype = i64
        L.por_chain_plane_len.argtypes = [C.c_int, sz]
        L.por_chain_nplanes.restype = C.c_int
        L.por_chain_nplanes.argtypes = [C.c_int]
        L.por_o1sac_decode.restype = i64
        L.por_o1sac_decode.argtypes = [vp, sz, C.c_uint, vp, sz, sz, vp, sz]
        L.por_o1sac_encode.restype = i64
        L.por_o1sac_encode.argtypes = [vp, sz, vp, sz, sz, vp, sz]
        for nm in ("por_int_delta", "por_predictor_xor", "por_mantissa_zero_strip"):
            getattr(L, nm).restype = C.c_int
            getattr(L, nm).argtypes = [vp, sz, C.c_uint, C.c_int, vp]
        for nm in ("por_reorder16_buf", "por_revert16_buf", "por_reorder32_buf", "por_revert32_buf"):
            getattr(L, nm).restype = None
            getattr(L, nm).argtypes = [vp, sz]
        L.por_byte_split.restype = None
        L.por_byte_split.argtypes = [vp, sz, C.c_int, vp]
        L.por_byte_merge.restype = None
        L.por_byte_merge.argtypes = [vp, sz, C.c_int, vp]
        L.por_nibble_split.restype = None
        L.por_nibble_split.argtypes = [vp, sz, vp, vp]
        L.por_nibble_merge.restype = None
        L.por_nibble_merge.argtypes = [vp, vp, sz, vp]
        for nm in ("por_reorder_e4m3", "por_revert_e4m3", "por_reorder_e5m2", "por_revert_e5m2"):
            getattr(L, nm).restype = C.c_uint8
            getattr(L, nm).argtypes = [C.c_uint8]
        for nm in ("por_reorder16x2", "por_revert16x2", "por_reorder32", "por_revert32"):
            getattr(L, nm).restype = C.c_uint32
            getattr(L, nm).argtypes = [C.c_uint32]
        L.por_crc32.restype = C.c_uint32
        L.por_crc32.argtypes = [C.c_uint32, vp, sz]
        L.por_xxh64.restype = C.c_uint64
        L.por_xxh64.argtypes = [vp, sz, C.c_uint64]
        L.por_blake3.restype = None
        L.por_blake3.argtypes = [vp, sz, vp]
        L.por_histogram.restype = None
        L.por_histogram.argtypes = [vp, sz, vp]
        _lib = L
    return _lib


def _buf(data) -> np.ndarray:
    if isinstance(data, np.ndarray):
        return np.ascontiguousarray(data).view(np.uint8).reshape(-1)
    return np.frombuffer(bytes(data), dtype=np.uint8)


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p) if a.size else None


# ---- entropy coders (raw blobs, entropy/{huffman,rans}) ----

def huf_compress(src, cap=None):
    """entropy/huffman/compress.rs:9 -> (outcome, blob)."""
    s = _buf(src)
    cap = cap if cap is not None else 2 * s.size + 4096
    dst = np.zeros(max(cap, 1), np.uint8)
    oc = C.c_int(0)
    n = lib().por_huf_compress(_ptr(dst), cap, _ptr(s), s.size, C.byref(oc))
    if n < 0:
        raise OracleError(n, "huf_compress")
    return oc.value, dst[:n].tobytes()


def huf_decompress(blob, n_out: int) -> bytes:
    b = _buf(blob)
    dst = np.zeros(max(n_out, 1), np.uint8)
    r = lib().por_huf_decompress(_ptr(dst), n_out, _ptr(b), b.size)
    if r < 0:
        raise OracleError(r, "huf_decompress")
    return dst[:n_out].tobytes()


def rans_compress(src, cap=None):
    s = _buf(src)
    cap = cap if cap is not None else 2 * s.size + 4096
    dst = np.zeros(max(cap, 1), np.uint8)
    oc = C.c_int(0)
    n = lib().por_rans_compress(_ptr(dst), cap, _ptr(s), s.size, C.byref(oc))
    if n < 0:
        raise OracleError(n, "rans_compress")
    return oc.value, dst[:n].tobytes()


def rans_decompress(blob, n_out: int) -> bytes:
    b = _buf(blob)
    dst = np.zeros(max(n_out, 1), np.uint8)
    r = lib().por_rans_decompress(_ptr(dst), n_out, _ptr(b), b.size)
    if r < 0:
        raise OracleError(r, "rans_decompress")
    return dst[:n_out].tobytes()


def zstd_decompress(blob, cap: int) -> bytes:
    """RFC 8878 frames (the zstd crate's decode_all, bounded by cap)."""
    b = _buf(blob)
    dst = np.zeros(max(cap, 1), np.uint8)
    r = lib().por_zstd_decompress(_ptr(dst), cap, _ptr(b), b.size)
    if r < 0:
        raise OracleError(r, "zstd_decompress")
    return dst[:r].tobytes()


def tans_compress(src) -> bytes:
    """entropy/tans/mod.rs:273 -> blob (b'' = store raw)."""
    s = _buf(src)
    dst = np.zeros(max(s.size, 1), np.uint8)
    n = lib().por_tans_compress(_ptr(dst), s.size, _ptr(s), s.size)
    if n < 0:
        raise OracleError(n, "tans_compress")
    return dst[:n].tobytes()


def tans_decompress(blob, n_out: int) -> bytes:
    """entropy/tans/mod.rs:372."""
    b = _buf(blob)
    dst = np.zeros(max(n_out, 1), np.uint8)
    r = lib().por_tans_decompress(_ptr(dst), n_out, _ptr(b), b.size)
    if r < 0:
        raise OracleError(r, "tans_decompress")
    return dst[:n_out].tobytes()


def tans_spread(norm):
    """entropy/tans/mod.rs:199 -> uint8[2048] slot symbols."""
    nm = np.ascontiguousarray(norm, np.uint32)
    t = np.zeros(2048, np.uint8)
    lib().por_tans_spread(_ptr(nm), _ptr(t))
    return t


def tans_decode_table(norm):
    """entropy/tans/mod.rs:346 -> (sym, nb_bits, baseline) arrays of 2048."""
    nm = np.ascontiguousarray(norm, np.uint32)
    sym = np.zeros(2048, np.uint8)
    nb = np.zeros(2048, np.uint8)
    base = np.zeros(2048, np.uint16)
    lib().por_tans_decode_table(_ptr(nm), _ptr(sym), _ptr(nb), _ptr(base))
    return sym, nb, base


# ---- plane codec payloads (codecs/{identity,huffman,rans}.rs) ----

def codec_encode(codec: int, plane) -> bytes:
    s = _buf(plane)
    cap = int(lib().por_codec_encode_bound(s.size))
    out = np.zeros(max(cap, 1), np.uint8)
    n = lib().por_codec_encode(codec, _ptr(s), s.size, _ptr(out), cap)
    if n < 0:
        raise OracleError(n, "codec_encode")
    return out[:n].tobytes()


# dispatch.rs:13-49 order of the codecs this oracle encodes (Identity last:
# priority 0 below the entropy coders' 1)
DEFAULT_MENU = (CODEC_HUFFMAN, CODEC_RANS, CODEC_TANS, CODEC_IDENTITY)


def select_encode(plane, menu=DEFAULT_MENU):
    """select.rs:27-64 trial encode -> (chosen codec, payload)."""
    s = _buf(plane)
    m = np.array(menu, np.uint16)
    cap = int(lib().por_codec_encode_bound(s.size))
    out = np.zeros(max(cap, 1), np.uint8)
    ch = np.zeros(1, np.uint16)
    n = lib().por_select_encode(_ptr(s), s.size, _ptr(m), m.size, _ptr(ch), _ptr(out), cap)
    if n < 0:
        raise OracleError(n, "select_encode")
    return int(ch[0]), out[:n].tobytes()


def codec_decode(codec: int, payload, cap: int) -> bytes:
    p = _buf(payload)
    out = np.zeros(max(cap, 1), np.uint8)
    n = lib().por_codec_decode(codec, _ptr(p), p.size, _ptr(out), cap)
    if n < 0:
        raise OracleError(n, "codec_decode")
    return out[:n].tobytes()


def encode_plane_chunked(codec: int, plane, chunk_size: int):
    """compressor.rs:324-381 -> (payload bytes, entries uint32[n,2])."""
    s = _buf(plane)
    cs = max(int(chunk_size), 1)
    nch = max(1, -(-s.size // cs))
    cap = nch * 5 + s.size + 5 * nch + 16
    out = np.zeros(cap, np.uint8)
    ent = np.zeros((nch, 2), np.uint32)
    nc = C.c_size_t(0)
    n = lib().por_encode_plane_chunked(codec, _ptr(s), s.size, cs, _ptr(out), cap, _ptr(ent), nch, C.byref(nc))
    if n < 0:
        raise OracleError(n, "encode_plane_chunked")
    return out[:n].tobytes(), ent[: nc.value].copy()


def decode_plane_chunked(codec: int, payload, entries, threads: int = 1) -> bytes:
    p = _buf(payload)
    ent = np.ascontiguousarray(entries, dtype=np.uint32)
    total = int(ent[:, 1].astype(np.uint64).sum()) if ent.size else 0
    out = np.zeros(max(total, 1), np.uint8)
    r = lib().por_decode_plane_chunked_mt(codec, _ptr(p), p.size, _ptr(ent), ent.shape[0], _ptr(out), total, threads)
    if r < 0:
        raise OracleError(r, "decode_plane_chunked")
    return out[:total].tobytes()


class TensorBatch:
    """Chunked plane payloads of several tensors of one chain and codec,
    decoded together by por_decode_tensors_mt (tensors over threads, chunks,
    fused inverse): the whole-container decode of container.rs:1766-2050."""

    def __init__(self, codec: int, chain: int, tensors):
        """tensors: iterable of (out_len, [(payload, entries) per plane])."""
        self.codec, self.chain = codec, chain
        np_ = lib().por_chain_nplanes(chain)
        self._keep = []
        pays, plens, ents, nents, outs, olens = [], [], [], [], [], []
        for out_len, planes in tensors:
            assert len(planes) == np_
            for pay, ent in planes:
                p = _buf(pay)
                e = np.ascontiguousarray(ent, dtype=np.uint32)
                self._keep += [p, e]
                pays.append(p.ctypes.data)
                plens.append(p.size)
                ents.append(e.ctypes.data)
                nents.append(e.shape[0])
            o = np.zeros(max(out_len, 1), np.uint8)
            self._keep.append(o)
            outs.append(o)
            olens.append(out_len)
        self.outs = outs
        self.out_lens = olens
        self.n = len(olens)
        self._pays = (C.c_void_p * len(pays))(*pays)
        self._plens = (C.c_size_t * len(plens))(*plens)
        self._ents = (C.c_void_p * len(ents))(*ents)
        self._nents = (C.c_size_t * len(nents))(*nents)
        self._outs = (C.c_void_p * self.n)(*[o.ctypes.data for o in outs])
        self._olens = (C.c_size_t * self.n)(*olens)

    def decode(self, threads: int) -> None:
        r = lib().por_decode_tensors_mt(self.codec, self.chain, self.n, self._pays, self._plens, self._ents,
                                        self._nents, self._outs, self._olens, threads)
        if r < 0:
            raise OracleError(r, "decode_tensors_mt")

    def output(self, i: int) -> bytes:
        return self.outs[i][: self.out_lens[i]].tobytes()


def _arr(ctype, vals):
    return (ctype * max(len(vals), 1))(*vals)


class PlaneBatch:
    """Tensors of any chain, each plane with its own codec, chunked or not,
    decoded together by por_batch_decode_mt: chunks of every plane over the
    threads (container.rs:1773,1996), then each tensor's inverse chain in
    slices.  The per-config CPU baseline of the bench."""

    def __init__(self, tensors):
        """tensors: iterable of (chain, out_len, [(codec, payload, entries or None) per plane])."""
        self._keep = []
        chains, olens, outs, codecs, pays, plens, ents, nents, bufs = [], [], [], [], [], [], [], [], []
        self.outs = []
        for chain, out_len, planes in tensors:
            pl = lib().por_chain_plane_len(chain, out_len)
            assert pl >= 0 and len(planes) == lib().por_chain_nplanes(chain)
            chains.append(chain)
            olens.append(out_len)
            o = np.zeros(max(out_len, 1), np.uint8)
            self.outs.append(o)
            outs.append(o.ctypes.data)
            for codec, pay, ent in planes:
                p = _buf(pay)
                e = np.zeros((0, 2), np.uint32) if ent is None else np.ascontiguousarray(ent, dtype=np.uint32)
                b = np.zeros(max(pl, 1), np.uint8)
                self._keep += [p, e, b]
                codecs.append(codec)
                pays.append(p.ctypes.data)
                plens.append(p.size)
                ents.append(e.ctypes.data)
                nents.append(e.shape[0])
                bufs.append(b.ctypes.data)
        self.out_lens = olens
        self.n = len(olens)
        self.restored = sum(olens)
        self._args = (self.n, _arr(C.c_int, chains), _arr(C.c_size_t, olens), _arr(C.c_void_p, outs),
                      _arr(C.c_int, codecs), _arr(C.c_void_p, pays), _arr(C.c_size_t, plens),
                      _arr(C.c_void_p, ents), _arr(C.c_size_t, nents), _arr(C.c_void_p, bufs))

    def decode(self, threads: int) -> None:
        r = lib().por_batch_decode_mt(*self._args, threads)
        if r < 0:
            raise OracleError(r, "batch_decode_mt")

    def output(self, i: int) -> bytes:
        return self.outs[i][: self.out_lens[i]].tobytes()


class PlaneBatchEncoder:
    """The encode direction of PlaneBatch (por_batch_encode_mt): the forward
    chain in slices, then every chunk of every plane over the threads."""

    def __init__(self, tensors):
        """tensors: iterable of (chain, raw bytes, [(codec, chunk_size or 0) per plane])."""
        self._keep = []
        chains, ilens, ins, codecs, csz, bufs, outs, ents = [], [], [], [], [], [], [], []
        self._planes = []
        for chain, raw, planes in tensors:
            r = _buf(raw)
            pl = lib().por_chain_plane_len(chain, r.size)
            assert pl >= 0 and len(planes) == lib().por_chain_nplanes(chain)
            self._keep.append(r)
            chains.append(chain)
            ilens.append(r.size)
            ins.append(r.ctypes.data)
            for codec, cs in planes:
                nch = max(1, -(-pl // cs)) if cs else 1
                cap = nch * (5 + lib().por_codec_encode_bound(cs)) if cs else lib().por_codec_encode_bound(pl)
                b = np.zeros(max(pl, 1), np.uint8)
                o = np.zeros(max(cap, 1), np.uint8)
                e = np.zeros((nch, 2), np.uint32)
                self._keep += [b, o, e]
                self._planes.append((o, e, cs))
                codecs.append(codec)
                csz.append(cs)
                bufs.append(b.ctypes.data)
                outs.append(o.ctypes.data)
                ents.append(e.ctypes.data)
        self.restored = sum(ilens)
        self._lens = (C.c_size_t * max(len(outs), 1))()
        self._args = (len(chains), _arr(C.c_int, chains), _arr(C.c_size_t, ilens), _arr(C.c_void_p, ins),
                      _arr(C.c_int, codecs), _arr(C.c_uint32, csz), _arr(C.c_void_p, bufs),
                      _arr(C.c_void_p, outs), _arr(C.c_void_p, ents), self._lens)

    def encode(self, threads: int) -> None:
        r = lib().por_batch_encode_mt(*self._args, threads)
        if r < 0:
            raise OracleError(r, "batch_encode_mt")

    def planes(self):
        """[(payload bytes, entries or None)] in plane order, after encode()."""
        return [(o[: self._lens[k]].tobytes(), e.copy() if cs else None)
                for k, (o, e, cs) in enumerate(self._planes)]


# ---- chains (transforms/fusion.rs) ----

def chain_forward(chain: int, data) -> list[bytes]:
    s = _buf(data)
    pl = int(lib().por_chain_plane_len(chain, s.size))
    if pl < 0:
        raise OracleError(-1, "chain_forward length")
    n = lib().por_chain_nplanes(chain)
    planes = [np.zeros(max(pl, 1), np.uint8) for _ in range(n)]
    ptrs = (C.c_void_p * n)(*[p.ctypes.data for p in planes])
    r = lib().por_chain_forward(chain, _ptr(s), s.size, ptrs)
    if r < 0:
        raise OracleError(r, "chain_forward")
    return [p[:pl].tobytes() for p in planes]


def chain_inverse(chain: int, planes) -> bytes:
    arrs = [_buf(p) for p in planes]
    n = lib().por_chain_nplanes(chain)
    assert len(arrs) == n and len({a.size for a in arrs}) == 1
    pl = arrs[0].size
    total = {CHAIN_IEEE16_SPLIT2: 2, CHAIN_IEEE32_SPLIT4: 4}.get(chain, 1) * pl
    out = np.zeros(max(total, 1), np.uint8)
    keep = [a if a.size else np.zeros(1, np.uint8) for a in arrs]
    ptrs = (C.c_void_p * n)(*[a.ctypes.data for a in keep])
    r = lib().por_chain_inverse(chain, ptrs, pl, _ptr(out))
    if r < 0:
        raise OracleError(r, "chain_inverse")
    return out[:total].tobytes()


# ---- Order1ScaleAC (codecs/order1_scale_ac.rs, range_coder.rs) ----

CODEC_O1SAC = 0x0011


def o1sac_decode(state, payload, n: int, row_len: int = 0, state_version: int = 1) -> bytes:
    """n symbols of an Order1ScaleAC payload under `state` (row_len 0: Flat)."""
    st, p = _buf(state), _buf(payload)
    out = np.zeros(max(n, 1), np.uint8)
    r = lib().por_o1sac_decode(_ptr(st), st.size, state_version, _ptr(p), p.size, row_len, _ptr(out), n)
    if r < 0:
        raise OracleError(r, "o1sac_decode")
    return out[:n].tobytes()


def o1sac_encode(state, plane, row_len: int = 0) -> bytes:
    st, s = _buf(state), _buf(plane)
    cap = 64 + 2 * s.size
    out = np.zeros(cap, np.uint8)
    r = lib().por_o1sac_encode(_ptr(st), st.size, _ptr(s), s.size, row_len, _ptr(out), cap)
    if r < 0:
        raise OracleError(r, "o1sac_encode")
    return out[:r].tobytes()


# ---- plane ops on one terminal plane (chain/dispatch.rs:96-122) ----

PLANE_OP_NONE = 0
PLANE_OP_INT_DELTA = 1
PLANE_OP_PREDICTOR_XOR = 2
PLANE_OP_MANTISSA_ZERO_STRIP = 3


def _plane_op(fn: str, data, param: int, inverse: bool) -> bytes:
    s = _buf(data)
    out = np.zeros(max(s.size, 1), np.uint8)
    r = getattr(lib(), fn)(_ptr(s), s.size, param, 1 if inverse else 0, _ptr(out))
    if r < 0:
        raise OracleError(r, fn)
    return out[: s.size].tobytes()


def int_delta(data, width: int = 1, inverse: bool = False) -> bytes:
    """transforms/int_delta.rs: wrapping delta at the element width (forward) or its running sum (inverse)."""
    return _plane_op("por_int_delta", data, width, inverse)


def predictor_xor(data, width: int = 1, inverse: bool = False) -> bytes:
    """transforms/predictor_xor.rs: fcm prediction residuals (forward) or the recovered values (inverse)."""
    return _plane_op("por_predictor_xor", data, width, inverse)


def mantissa_zero_strip(data, k: int, inverse: bool = False) -> bytes:
    """transforms/mantissa_zero.rs: b >> k (forward, refused on nonzero low bits) or b << k (inverse)."""
    return _plane_op("por_mantissa_zero_strip", data, k, inverse)


def plane_op(op: int, param: int, data, inverse: bool) -> bytes:
    """One plane op by its PTMD code (PLANE_OP_*): param = width (deltas) or k (strip)."""
    if op == PLANE_OP_NONE:
        return bytes(data)
    fn = {PLANE_OP_INT_DELTA: int_delta, PLANE_OP_PREDICTOR_XOR: predictor_xor,
          PLANE_OP_MANTISSA_ZERO_STRIP: mantissa_zero_strip}[op]
    return fn(data, param, inverse)


# ---- chain trial (compressor.rs:504-640) over the split chains' plane-op variants ----

def split_chain_variants(chain: int):
    """The production split-chain variants that stay within the plane codec
    (python/ptwm/preprocessing/_chains.py:1146-1185 order): per variant the
    (op, param) of every plane.  Exponent plane: 1 (bf16/fp16), 3 (fp32);
    MantissaZeroStrip on plane 0."""
    np_ = 2 if chain == CHAIN_IEEE16_SPLIT2 else 4
    ex = 1 if chain == CHAIN_IEEE16_SPLIT2 else 3
    none = [(PLANE_OP_NONE, 0)] * np_
    out = [list(none)]
    for op in (PLANE_OP_INT_DELTA, PLANE_OP_PREDICTOR_XOR):
        v = list(none)
        v[ex] = (op, 1)
        out.append(v)
    for k in range(1, 5):
        v = list(none)
        v[0] = (PLANE_OP_MANTISSA_ZERO_STRIP, k)
        out.append(v)
    return out


def chain_trial(chain: int, data, menu):
    """pass1_select_chain (compressor.rs:504-640): every variant forward and
    every terminal trial-encoded over `menu` (select.rs:27-64); the first
    variant with the smallest total payload wins; a variant whose forward
    fails is skipped.  Returns (variant ops, [(codec, payload)] per plane)."""
    planes = chain_forward(chain, data)
    best = None
    for ops in split_chain_variants(chain):
        try:
            terms = [plane_op(op, prm, pl, inverse=False) for (op, prm), pl in zip(ops, planes)]
        except OracleError:
            continue
        enc = [select_encode(t, menu) for t in terms]
        total = sum(len(e[1]) for e in enc)
        if best is None or total < best[0]:
            best = (total, ops, enc)
    return best[1], best[2]


# ---- Huffman internals ----

def huf_lengths(freqs):
    f = np.ascontiguousarray(freqs, dtype=np.uint32)
    assert f.size == 256
    lengths = np.zeros(256, np.uint8)
    ok = lib().por_huf_lengths_from_freqs(_ptr(f), _ptr(lengths))
    return lengths if ok else None


def huf_lengths_limited(freqs, max_len):
    """The reference tree with enforce_max_code_length at max_len."""
    f = np.ascontiguousarray(freqs, dtype=np.uint32)
    assert f.size == 256
    lengths = np.zeros(256, np.uint8)
    ok = lib().por_huf_lengths_limited(_ptr(f), _ptr(lengths), int(max_len))
    return lengths if ok else None


def ilv_lengths(freqs):
    """huff_ilv encoder code lengths (limit 6 for nibble alphabets, else 11)."""
    f = np.ascontiguousarray(freqs, dtype=np.uint32)
    assert f.size == 256
    lengths = np.zeros(256, np.uint8)
    ok = lib().por_ilv_lengths(_ptr(f), _ptr(lengths))
    return lengths if ok else None


def huf_table(lengths):
    """tree.rs:102-177 -> (max_bits, decode_table, rev_codes) or None."""
    l8 = np.ascontiguousarray(lengths, dtype=np.uint8)
    assert l8.size == 256
    table = np.zeros(2048, np.uint16)
    rev = np.zeros(256, np.uint16)
    mb = lib().por_huf_from_lengths(_ptr(l8), _ptr(table), _ptr(rev))
    if mb == 0:
        return None
    return mb, table[: 1 << mb].copy(), rev


def huf_encode_weights(weights) -> bytes:
    w = _buf(weights)
    out = np.zeros(260, np.uint8)
    n = lib().por_huf_encode_weights(_ptr(w), w.size, _ptr(out), out.size)
    if n < 0:
        raise OracleError(n, "encode_weights")
    return out[:n].tobytes()


def huf_decode_weights(src):
    s = _buf(src)
    w = np.zeros(256, np.uint8)
    nn = C.c_int(0)
    used = lib().por_huf_decode_weights(_ptr(s), s.size, _ptr(w), C.byref(nn))
    if used < 0:
        raise OracleError(used, "decode_weights")
    return w[: nn.value].tobytes(), int(used)


def bitwriter_pack(codes) -> bytes:
    bits = np.array([c[0] for c in codes], np.uint16)
    nb = np.array([c[1] for c in codes], np.uint8)
    out = np.zeros(len(codes) * 2 + 16, np.uint8)
    n = lib().por_bitwriter_pack(_ptr(bits), _ptr(nb), len(codes), _ptr(out), out.size)
    if n < 0:
        raise OracleError(n, "bitwriter_pack")
    return out[:n].tobytes()


def rans_normalize(raw):
    r = np.ascontiguousarray(raw, dtype=np.uint32)
    f = np.zeros(256, np.uint16)
    cum = np.zeros(256, np.uint16)
    ok = lib().por_rans_normalize(_ptr(r), _ptr(f), _ptr(cum))
    return (f, cum) if ok else None


# ---- integrity ----

def crc32(data, crc: int = 0) -> int:
    b = _buf(data)
    return int(lib().por_crc32(crc, _ptr(b), b.size))


def xxh64(data, seed: int = 0) -> int:
    b = _buf(data)
    return int(lib().por_xxh64(_ptr(b), b.size, seed))


def blake3(data) -> bytes:
    b = _buf(data)
    out = np.zeros(32, np.uint8)
    lib().por_blake3(_ptr(b), b.size, _ptr(out))
    return out.tobytes()


def histogram(data):
    b = _buf(data)
    h = np.zeros(256, np.uint32)
    lib().por_histogram(_ptr(b), b.size, _ptr(h))
    return h


# ---- huff_ilv (this build's own codec; the functions are its spec) ----

def ilv_encode(plane) -> bytes:
    L = lib()
    L.por_ilv_encode.restype = C.c_int64
    L.por_ilv_encode.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t]
    L.por_ilv_encode_bound.restype = C.c_size_t
    L.por_ilv_encode_bound.argtypes = [C.c_size_t]
    s = _buf(plane)
    cap = int(L.por_ilv_encode_bound(s.size))
    out = np.zeros(cap, np.uint8)
    n = L.por_ilv_encode(_ptr(s), s.size, _ptr(out), cap)
    if n < 0:
        raise OracleError(n, "ilv_encode")
    return out[:n].tobytes()


def ilv_decode(payload, cap: int) -> bytes:
    L = lib()
    L.por_ilv_decode.restype = C.c_int64
    L.por_ilv_decode.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t]
    p = _buf(payload)
    out = np.zeros(max(cap, 1), np.uint8)
    n = L.por_ilv_decode(_ptr(p), p.size, _ptr(out), cap)
    if n < 0:
        raise OracleError(n, "ilv_decode")
    return out[:n].tobytes()


def ilv_encode_coded(plane) -> bytes:
    """The huff_ilv coded form (tag 1) of a plane whatever its size: test
    payloads that no encoder would choose but every decoder must accept."""
    L = lib()
    L.por_ilv_encode_coded.restype = C.c_int64
    L.por_ilv_encode_coded.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t]
    L.por_ilv_encode_bound.restype = C.c_size_t
    L.por_ilv_encode_bound.argtypes = [C.c_size_t]
    s = _buf(plane)
    cap = int(L.por_ilv_encode_bound(s.size)) + 4096
    out = np.zeros(cap, np.uint8)
    n = L.por_ilv_encode_coded(_ptr(s), s.size, _ptr(out), cap)
    if n < 0:
        raise OracleError(n, "ilv_encode_coded")
    return out[:n].tobytes()


def rans_ilv_encode(plane) -> bytes:
    """rans_ilv (this build's GPU-native interleaved rANS codec) payload of
    a plane: the format's specification (por_rans_ilv_encode)."""
    L = lib()
    L.por_rans_ilv_encode.restype = C.c_int64
    L.por_rans_ilv_encode.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t]
    s = _buf(plane)
    cap = s.size + 1
    out = np.zeros(cap, np.uint8)
    n = L.por_rans_ilv_encode(_ptr(s), s.size, _ptr(out), cap)
    if n < 0:
        raise OracleError(n, "rans_ilv_encode")
    return out[:n].tobytes()


def rans_ilv_encode_coded(plane) -> bytes:
    """The rans_ilv coded form (tag 1) of a plane whatever its size (test
    payloads, as ilv_encode_coded)."""
    L = lib()
    L.por_rans_ilv_encode_coded.restype = C.c_int64
    L.por_rans_ilv_encode_coded.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t]
    s = _buf(plane)
    cap = 2 * s.size + 65536
    out = np.zeros(cap, np.uint8)
    n = L.por_rans_ilv_encode_coded(_ptr(s), s.size, _ptr(out), cap)
    if n < 0:
        raise OracleError(n, "rans_ilv_encode_coded")
    return out[:n].tobytes()


def rans_ilv_decode(payload, cap: int) -> bytes:
    L = lib()
    L.por_rans_ilv_decode.restype = C.c_int64
    L.por_rans_ilv_decode.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t]
    p = _buf(payload)
    out = np.zeros(max(cap, 1), np.uint8)
    n = L.por_rans_ilv_decode(_ptr(p), p.size, _ptr(out), cap)
    if n < 0:
        raise OracleError(n, "rans_ilv_decode")
    return out[:n].tobytes()
