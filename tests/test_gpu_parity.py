"""GPU parity: the HIP path against the CPU oracle, through the C ABI.

Bit-exact on every case.  Encoded inputs come from the oracle (a C
restatement of the reference encoder), so GPU decode is checked on
reference-format streams; malformed payloads must be rejected exactly where
the oracle (reference decoder state machine) rejects them.
"""
import os
import sys

import numpy as np
import pytest

import oracle as O
from ptwm_amd import api, ids, plan

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

SEL = ids.PLANE_CODEC_LABEL
BACKEND = ids.HARDWARE_BACKEND_LABEL
PLAN_ID = ids.DECODE_PLAN_LABEL


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dev(b: bytes, pad: int = 0):
    a = np.frombuffer(bytes(b), np.uint8)
    t = torch.zeros(max(len(a) + pad, 1), dtype=torch.uint8, device="cuda:0")
    if len(a):
        t[: len(a)].copy_(torch.from_numpy(a.copy()))
    return t[: len(a) + pad] if len(a) + pad > 0 else t[:0]


def host(t) -> bytes:
    torch.cuda.synchronize()
    return t.cpu().numpy().tobytes()


CODEC_NAME = {O.CODEC_IDENTITY: "identity", O.CODEC_HUFFMAN: "huffman", O.CODEC_RANS: "rans"}


def gpu_decode(codec, payload: bytes, cap: int):
    src = dev(payload)
    dst = torch.zeros(max(cap, 1), dtype=torch.uint8, device="cuda:0")[:cap]
    try:
        n = api.plane_codec_decode_cuda(SEL, CODEC_NAME[codec], b"", src, dst, 0)
    except Exception as e:  # noqa: BLE001
        return getattr(e, "rc", -99), None
    return n, host(dst)[:n]


def oracle_decode(codec, payload: bytes, cap: int):
    try:
        return 0, O.codec_decode(codec, payload, cap)
    except O.OracleError as e:
        return e.rc, None


def data_cases():
    rng = np.random.default_rng(42)
    yield "empty", b""
    yield "one", b"\x07"
    for n in (2, 3, 4, 5, 7, 8, 15, 16, 17, 63, 64, 65):
        yield f"skew{n}", bytes(rng.geometric(0.5, n).clip(0, 255).astype(np.uint8))
    yield "mod64", bytes(i % 64 for i in range(4096))
    yield "odd4093", bytes(i % 50 for i in range(4093))
    yield "single", bytes([42]) * 1024
    yield "two", bytes([0] * 3000 + [1] * 1000)
    yield "high", bytes([0] * 3000 + [200] * 600 + [128] * 200 + [255] * 100)
    yield "uniform", bytes(range(256)) * 4
    yield "geo64k", bytes(rng.geometric(0.25, 65536).clip(0, 255).astype(np.uint8))
    w = (torch.randn(256 * 1024, generator=torch.Generator().manual_seed(1)) * 0.02).to(torch.bfloat16)
    yield "bf16exp", np.frombuffer(O.chain_forward(O.CHAIN_IEEE16_SPLIT2, w.view(torch.uint8).numpy().tobytes())[1], np.uint8).tobytes()
    yield "skewed256", bytes(np.where(rng.random(50000) < 0.9, 0, rng.integers(1, 256, 50000)).astype(np.uint8))


@pytest.mark.parametrize("codec", [O.CODEC_IDENTITY, O.CODEC_HUFFMAN, O.CODEC_RANS])
def test_decode_reference_payloads(codec):
    for name, src in data_cases():
        note(f"decode codec={codec} case={name} n={len(src)}")
        payload = O.codec_encode(codec, src)
        n, out = gpu_decode(codec, payload, len(src))
        assert n == len(src), (name, n)
        assert out == src, name


@pytest.mark.parametrize("codec", [O.CODEC_HUFFMAN, O.CODEC_RANS])
def test_decode_malformed_matches_reference(codec):
    """Corrupt / truncated / extended payloads: accept and reject exactly as
    the reference decoder does, with identical bytes when accepted."""
    rng = np.random.default_rng(7 + codec)
    bases = [bytes(i % 64 for i in range(4096)), bytes(rng.geometric(0.3, 3001).clip(0, 255).astype(np.uint8)),
             bytes([0, 0, 0, 1] * 64)]
    n_checked = 0
    for bi, src in enumerate(bases):
        good = O.codec_encode(codec, src)
        variants = []
        for k in range(60):
            b = bytearray(good)
            kind = k % 5
            if kind == 0:
                i = int(rng.integers(5, len(b)))
                b[i] ^= int(rng.integers(1, 256))
            elif kind == 1:
                b = b[: int(rng.integers(1, len(b)))]
            elif kind == 2:
                i = int(rng.integers(5, len(b)))
                b[i:i] = bytes([int(rng.integers(0, 256))])
            elif kind == 3:
                for _ in range(4):
                    i = int(rng.integers(5, len(b)))
                    b[i] = int(rng.integers(0, 256))
            else:
                i = int(rng.integers(5, min(len(b), 40)))
                b[i] ^= 1 << int(rng.integers(0, 8))
            variants.append(bytes(b))
        for vi, v in enumerate(variants):
            cap = len(src)
            note(f"malformed codec={codec} base={bi} variant={vi}")
            rc_o, out_o = oracle_decode(codec, v, cap)
            n_g, out_g = gpu_decode(codec, v, cap)
            if rc_o < 0:
                assert n_g < 0, (bi, vi)
            else:
                assert n_g == len(out_o) and out_g == out_o, (bi, vi)
            n_checked += 1
    assert n_checked == 180


CHAINS = [(O.CHAIN_IEEE16_SPLIT2, 2), (O.CHAIN_IEEE32_SPLIT4, 4), (O.CHAIN_E4M3_NIBBLE, 1),
          (O.CHAIN_E5M2_NIBBLE, 1), (O.CHAIN_NIBBLE_SPLIT, 1), (O.CHAIN_PASSTHROUGH, 1)]


@pytest.mark.parametrize("chain,unit", CHAINS)
@pytest.mark.parametrize("n_elems", [1, 15, 16, 17, 255, 4096, 100003])
def test_split_merge_match_oracle(chain, unit, n_elems):
    note(f"split/merge chain={chain} n={n_elems}")
    rng = np.random.default_rng(n_elems + 31 * chain)
    data = rng.integers(0, 256, n_elems * unit, dtype=np.uint8).tobytes()
    want_planes = O.chain_forward(chain, data)
    src = dev(data)
    planes = [torch.zeros(len(want_planes[0]), dtype=torch.uint8, device="cuda:0") for _ in want_planes]
    n = api.split_cuda(chain, src, planes)
    assert n == len(want_planes[0])
    for p, w in zip(planes, want_planes):
        assert host(p) == w
    out = torch.zeros(len(data), dtype=torch.uint8, device="cuda:0")
    # merge from planes with dirty high nibbles for nibble chains (masked on inverse)
    if chain in (O.CHAIN_E4M3_NIBBLE, O.CHAIN_E5M2_NIBBLE, O.CHAIN_NIBBLE_SPLIT):
        planes = [p | torch.tensor(0xF0, dtype=torch.uint8, device="cuda:0") for p in planes]
    assert api.merge_cuda(chain, planes, out) == len(data)
    assert host(out) == data


def build_tensor(chain, data: bytes, codecs, chunk_size=None, base_offset=0):
    """Encode a tensor with the oracle; return (payload bytes, TensorPlan)."""
    planes = O.chain_forward(chain, data)
    blob = bytearray()
    pls = []
    for p, codec in zip(planes, codecs):
        while (base_offset + len(blob)) % 16:
            blob += b"\xee"
        off = base_offset + len(blob)
        if chunk_size:
            payload, ent = O.encode_plane_chunked(codec, p, chunk_size)
            chunks = [(int(a), int(b)) for a, b in ent]
        else:
            payload = O.codec_encode(codec, p)
            chunks = None
        blob += payload
        pls.append(plan.PlanePlan(codec, off, len(payload), len(p), chunks))
    return bytes(blob), plan.TensorPlan(chain, 0, len(data), pls)


def gpu_tensor_decode(blob: bytes, tensors, out_len):
    st = plan.encode_plan(tensors)
    src = dev(blob)
    out = torch.zeros(max(out_len, 1), dtype=torch.uint8, device="cuda:0")[:out_len]
    n = api.hardware_backend_dispatch_decode_cuda(BACKEND, PLAN_ID, st, src, out, 0)
    return n, host(out)


def bf16_bytes(n, seed, std=0.02):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n, generator=g) * std).to(torch.bfloat16).view(torch.uint8).numpy().tobytes()


@pytest.mark.parametrize("chunk", [None, 4096, 65536])
@pytest.mark.parametrize("codecs", [(0, 1), (1, 1), (0, 3), (3, 3)])
def test_tensor_decode_bf16(chunk, codecs):
    note(f"tensor bf16 chunk={chunk} codecs={codecs}")
    data = bf16_bytes(100_000, 3)
    blob, t = build_tensor(O.CHAIN_IEEE16_SPLIT2, data, codecs, chunk)
    n, out = gpu_tensor_decode(blob, [t], len(data))
    assert n == len(data) and out == data


def test_tensor_decode_config1_bf16_1024x1024():
    """bf16 1024x1024 N(0, 0.02), 2-plane split, Huffman."""
    note("config1")
    data = bf16_bytes(1024 * 1024, 1)
    blob, t = build_tensor(O.CHAIN_IEEE16_SPLIT2, data, (O.CODEC_HUFFMAN, O.CODEC_HUFFMAN))
    n, out = gpu_tensor_decode(blob, [t], len(data))
    assert n == len(data) and out == data


def test_tensor_decode_fp32_outliers_chunked():
    """Config 2 shape reduced to 512x512: fp32 N(0,0.02) with 1% x50 outliers,
    4-plane split, rANS exponent plane, Huffman mantissa planes, 256 KiB
    chunks (the full 4096x4096 case runs in bench.py)."""
    note("config2-small")
    g = torch.Generator().manual_seed(2)
    w = torch.randn(512, 512, generator=g) * 0.02
    m = torch.rand(512, 512, generator=g) < 0.01
    w[m] *= 50
    data = w.numpy().tobytes()
    blob, t = build_tensor(O.CHAIN_IEEE32_SPLIT4, data, (1, 1, 1, 3), 65536)
    n, out = gpu_tensor_decode(blob, [t], len(data))
    assert n == len(data) and out == data


@pytest.mark.parametrize("codec", [O.CODEC_HUFFMAN, O.CODEC_RANS])
def test_tensor_decode_fp8_e4m3(codec):
    note(f"fp8 codec={codec}")
    g = torch.Generator().manual_seed(3)
    x = torch.randn(256, 1024, generator=g)
    x = x / x.abs().amax(1, keepdim=True) * 448
    data = x.to(torch.float8_e4m3fn).view(torch.uint8).numpy().tobytes()
    blob, t = build_tensor(O.CHAIN_E4M3_NIBBLE, data, (codec, codec), 65536)
    n, out = gpu_tensor_decode(blob, [t], len(data))
    assert n == len(data) and out == data


def test_tensor_decode_mxfp4_weights_and_scales_multi_tensor():
    """Config 5 shape reduced: u8 weights (two FP4 nibbles) nibble-split +
    E8M0 scales passthrough, two tensors in one plan."""
    note("config5-small")
    rng = np.random.default_rng(5)
    w = (rng.integers(0, 16, (1024, 256)) | (rng.integers(0, 16, (1024, 256)) << 4)).astype(np.uint8).tobytes()
    s = np.clip(np.round(rng.normal(-6, 1.5, (1024, 16))) + 127, 0, 255).astype(np.uint8).tobytes()
    blob_w, tw = build_tensor(O.CHAIN_NIBBLE_SPLIT, w, (O.CODEC_HUFFMAN, O.CODEC_RANS), 65536)
    blob_s, ts = build_tensor(O.CHAIN_PASSTHROUGH, s, (O.CODEC_HUFFMAN,), None, base_offset=len(blob_w))
    ts.out_offset = len(w)
    n, out = gpu_tensor_decode(blob_w + blob_s, [tw, ts], len(w) + len(s))
    assert n == len(w) + len(s) and out == w + s


def test_tensor_decode_rejects_corrupt_chunk():
    note("corrupt chunk")
    data = bf16_bytes(50_000, 9)
    blob, t = build_tensor(O.CHAIN_IEEE16_SPLIT2, data, (1, 1), 8192)
    b = bytearray(blob)
    off = t.planes[1].payload_offset + t.planes[1].chunks[2][0]
    b[off + 1] = 0xFF   # state_len past the frame
    with pytest.raises(Exception):
        gpu_tensor_decode(bytes(b), [t], len(data))
