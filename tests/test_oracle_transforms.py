"""Oracle checks: bit reorder, byte/nibble split, fused chains.

Pinned by the reference's known answers (cited per test), exhaustive
bijection over every fp8 / 16-bit value, and fused == unfused composition
(transforms/fusion.rs:525-751 asserts the same identity).
"""
import numpy as np
import pytest

import oracle as O


def test_e4m3_known_answers(orc):
    # split/dtype8.rs:211-235
    L = orc.lib()
    assert L.por_reorder_e4m3(0x38) == 0x70 and L.por_revert_e4m3(0x70) == 0x38
    assert L.por_reorder_e4m3(0x7E) == 0xF6 and L.por_revert_e4m3(0xF6) == 0x7E
    assert L.por_reorder_e4m3(0xB8) == 0x78 and L.por_revert_e4m3(0x78) == 0xB8


def test_e5m2_known_answers(orc):
    # split/dtype8.rs:238-249
    L = orc.lib()
    assert L.por_reorder_e5m2(0x3C) == 0x78 and L.por_revert_e5m2(0x78) == 0x3C
    assert L.por_reorder_e5m2(0xBC) == 0x7C and L.por_revert_e5m2(0x7C) == 0xBC


def test_fp8_reorder_exhaustive_semantics(orc):
    # exponent field lands in the high nibble (E4M3) / top 5 bits (E5M2):
    # checked from the IEEE field definitions, not from the oracle formula.
    L = orc.lib()
    seen4, seen5 = set(), set()
    for v in range(256):
        s, e4, m3 = v >> 7, (v >> 3) & 0xF, v & 7
        r = L.por_reorder_e4m3(v)
        assert r >> 4 == e4 and (r >> 3) & 1 == s and r & 7 == m3
        assert L.por_revert_e4m3(r) == v
        e5, m2 = (v >> 2) & 0x1F, v & 3
        r5 = L.por_reorder_e5m2(v)
        assert r5 >> 3 == e5 and (r5 >> 2) & 1 == s and r5 & 3 == m2
        assert L.por_revert_e5m2(r5) == v
        seen4.add(r); seen5.add(r5)
    assert len(seen4) == 256 and len(seen5) == 256


def test_ieee16_reorder_field_semantics(orc):
    # [S E8 M7] -> [E8 S M7] per 16-bit half (split/dtype16.rs:6-24)
    L = orc.lib()
    vals = np.arange(65536, dtype=np.uint32)
    outs = set()
    for v in range(0, 65536, 7):
        w = v | ((65535 - v) << 16)
        r = L.por_reorder16x2(w)
        for half, hv in ((r & 0xFFFF, v), (r >> 16, 65535 - v)):
            s, e, m = hv >> 15, (hv >> 7) & 0xFF, hv & 0x7F
            assert half >> 8 == e and (half >> 7) & 1 == s and half & 0x7F == m
        assert L.por_revert16x2(r) == w
        outs.add(r & 0xFFFF)
    assert len(outs) == len(range(0, 65536, 7))
    del vals


def test_ieee32_reorder_field_semantics(orc):
    L = orc.lib()
    rng = np.random.default_rng(0)
    for v in list(rng.integers(0, 2**32, 5000, dtype=np.uint64)) + [0, 2**32 - 1, 0x80000000, 0x7F800000]:
        v = int(v)
        r = L.por_reorder32(v)
        s, e, m = v >> 31, (v >> 23) & 0xFF, v & 0x7FFFFF
        assert r >> 24 == e and (r >> 23) & 1 == s and r & 0x7FFFFF == m
        assert L.por_revert32(r) == v


def test_byte_split_interleave_known_answer(orc):
    # transforms/byte_split.rs:302-313: [0,1,2,3] n=2 -> [0,2],[1,3]
    src = np.array([0, 1, 2, 3], np.uint8)
    p0, p1 = np.zeros(2, np.uint8), np.zeros(2, np.uint8)
    import ctypes as C
    ptrs = (C.c_void_p * 2)(p0.ctypes.data, p1.ctypes.data)
    orc.lib().por_byte_split(src.ctypes.data, 4, 2, ptrs)
    assert p0.tolist() == [0, 2] and p1.tolist() == [1, 3]


@pytest.mark.parametrize("n", [2, 4, 8])
def test_byte_split_roundtrip(orc, n):
    import ctypes as C
    rng = np.random.default_rng(n)
    data = rng.integers(0, 256, 64 * n, dtype=np.uint8)
    planes = [np.zeros(64, np.uint8) for _ in range(n)]
    ptrs = (C.c_void_p * n)(*[p.ctypes.data for p in planes])
    orc.lib().por_byte_split(data.ctypes.data, data.size, n, ptrs)
    for i in range(n):
        assert np.array_equal(planes[i], data[i::n])
    out = np.zeros_like(data)
    orc.lib().por_byte_merge(ptrs, 64, n, out.ctypes.data)
    assert np.array_equal(out, data)


def test_nibble_split_known_answers(orc):
    # transforms/nibble_split.rs:222-276
    hi, lo = np.zeros(1, np.uint8), np.zeros(1, np.uint8)
    orc.lib().por_nibble_split(np.array([0xAB], np.uint8).ctypes.data, 1, hi.ctypes.data, lo.ctypes.data)
    assert hi[0] == 0x0A and lo[0] == 0x0B
    # dirty high bits are masked by the inverse
    h = np.array([0xFA, 0xFB], np.uint8); l_ = np.array([0x0C, 0x0D], np.uint8)
    out = np.zeros(2, np.uint8)
    orc.lib().por_nibble_merge(h.ctypes.data, l_.ctypes.data, 2, out.ctypes.data)
    assert out.tolist() == [0xAC, 0xBD]


@pytest.mark.parametrize("chain,unit", [(O.CHAIN_IEEE16_SPLIT2, 2), (O.CHAIN_IEEE32_SPLIT4, 4),
                                        (O.CHAIN_E4M3_NIBBLE, 1), (O.CHAIN_E5M2_NIBBLE, 1),
                                        (O.CHAIN_NIBBLE_SPLIT, 1), (O.CHAIN_PASSTHROUGH, 1)])
@pytest.mark.parametrize("n_elems", [0, 1, 2, 3, 5, 64, 1023])
def test_fused_equals_unfused(orc, chain, unit, n_elems):
    """fusion.rs:525-751: fused forward == reorder op then split op; inverse roundtrips."""
    rng = np.random.default_rng(n_elems * 7 + chain)
    data = rng.integers(0, 256, n_elems * unit, dtype=np.uint8).tobytes()
    planes = O.chain_forward(chain, data)
    b = np.frombuffer(data, np.uint8)
    if chain == O.CHAIN_IEEE16_SPLIT2:
        v = b.view(np.uint16).astype(np.uint32)
        r = (((v << 1) & 0xFF00) | ((v >> 8) & 0x80) | (v & 0x7F)).astype(np.uint16)
        rb = r.view(np.uint8)
        exp = [rb[0::2].tobytes(), rb[1::2].tobytes()]
    elif chain == O.CHAIN_IEEE32_SPLIT4:
        v = b.view(np.uint32).astype(np.uint64)
        r = (((v << 1) & 0xFF000000) | ((v >> 8) & 0x800000) | (v & 0x7FFFFF)).astype(np.uint32)
        rb = r.view(np.uint8)
        exp = [rb[i::4].tobytes() for i in range(4)]
    elif chain in (O.CHAIN_E4M3_NIBBLE, O.CHAIN_E5M2_NIBBLE):
        f = orc.lib().por_reorder_e4m3 if chain == O.CHAIN_E4M3_NIBBLE else orc.lib().por_reorder_e5m2
        r = np.array([f(int(x)) for x in b], np.uint8)
        exp = [(r >> 4).tobytes(), (r & 15).tobytes()]
    elif chain == O.CHAIN_NIBBLE_SPLIT:
        exp = [(b >> 4).tobytes(), (b & 15).tobytes()]
    else:
        exp = [data]
    assert planes == exp
    assert O.chain_inverse(chain, planes) == data


def test_unfused_ieee16_leaves_odd_trailing_element(orc):
    """split/dtype16.rs:31-47 reorders whole u32 words only; the fused op
    (fusion.rs:73-89) reorders the trailing element too."""
    data = np.array([0x12, 0xC3, 0x45, 0xB6, 0x78, 0xC9], np.uint8)
    un = data.copy()
    orc.lib().por_reorder16_buf(un.ctypes.data, un.size)
    assert un[4:].tolist() == [0x78, 0xC9]
    fused = O.chain_forward(O.CHAIN_IEEE16_SPLIT2, data.tobytes())
    v = 0xC978
    r = ((v << 1) & 0xFF00) | ((v >> 8) & 0x80) | (v & 0x7F)
    assert fused[0][2] == (r & 0xFF) and fused[1][2] == (r >> 8)


def test_chain_rejects_bad_lengths(orc):
    assert orc.lib().por_chain_plane_len(O.CHAIN_IEEE16_SPLIT2, 3) == -1
    assert orc.lib().por_chain_plane_len(O.CHAIN_IEEE32_SPLIT4, 6) == -1
