"""Inverse plane ops on the device (IntDelta, PredictorXor, MantissaZeroStrip)
against the oracle.

The reference's production split chains put one op on one terminal plane
(python/ptwm/preprocessing/_chains.py:360-600): IntDelta or PredictorXor on
the exponent plane, MantissaZeroStrip(k) on the (low) mantissa plane.  The
decode runs the op's inverse on the decoded plane after its CRC check and
before the merge (container.rs:2152-2170).  Plans here are built from the
oracle's forward ops and codecs, decoded through the tensor-level entry
point, and compared with the oracle's plan decode (tests/plan_oracle.py),
which checks the same CRCs and hashes.  The reference's own smooth-data
frames (IntDelta) run through tests/test_gpu_container.py.
"""
import sys

import numpy as np
import pytest

import oracle as O
from ptwm_amd import api, ids, plan as P

import plan_oracle

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dev_bytes(b: bytes):
    t = torch.empty(max(1, len(b)), dtype=torch.uint8, device="cuda:0")
    if b:
        t[: len(b)].copy_(torch.from_numpy(np.frombuffer(b, np.uint8).copy()))
    return t[: len(b)]


def dispatch(state: bytes, blob: bytes, out_len: int):
    src = dev_bytes(blob)
    out = torch.full((max(out_len, 1),), 0xA5, dtype=torch.uint8, device="cuda:0")
    n = api.hardware_backend_dispatch_decode_cuda(ids.HARDWARE_BACKEND_LABEL, ids.DECODE_PLAN_LABEL, state, src,
                                                  out[:out_len], 0)
    torch.cuda.synchronize()
    return n, out[:out_len].cpu().numpy().tobytes()


def encode_payload(codec, plane):
    if codec == 0x7F01:
        return O.ilv_encode(plane)
    return O.codec_encode(codec, plane)


def build(tensors, with_crc=True, with_hash=True):
    """tensors: (chain, raw bytes, [(codec, op, param)] per plane).  Returns
    (plan bytes, input blob, out_len, raws)."""
    blob = bytearray()
    tplans = []
    out_off = 0
    for chain, raw, spec in tensors:
        planes = O.chain_forward(chain, raw)
        pps = []
        for plane, (codec, op, param) in zip(planes, spec):
            term = plane if op == P.PLANE_OP_NONE else O.plane_op(op, param, plane, inverse=False)
            pay = encode_payload(codec, term)
            off = (len(blob) + 255) // 256 * 256
            blob += b"\0" * (off - len(blob)) + pay
            pps.append(P.PlanePlan(codec, off, len(pay), len(term), None, O.crc32(term) if with_crc else None,
                                   op, param))
        tplans.append(P.TensorPlan(chain, out_off, len(raw), pps, O.xxh64(raw) if with_hash else None))
        out_off = (out_off + len(raw) + 255) // 256 * 256
    return P.encode_plan(tplans), bytes(blob), out_off, [t[1] for t in tensors]


def bf16_tensor(n, seed, smooth=False):
    g = torch.Generator().manual_seed(seed)
    if smooth:
        x = torch.cumsum(torch.randn(n, generator=g) * 0.01, 0) + torch.linspace(-3, 3, n)
    else:
        x = torch.randn(n, generator=g) * 0.02
    return x.to(torch.bfloat16).view(torch.uint8).numpy().tobytes()


def fp32_tensor(n, seed, quant_bits=0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.cumsum(torch.randn(n, generator=g) * 0.01, 0)).to(torch.float32)
    v = x.view(torch.int32)
    if quant_bits:
        v = v & ~((1 << quant_bits) - 1)  # low mantissa bits cleared: the strip applies
    return v.numpy().tobytes()


def check(tensors, **kw):
    state, blob, out_len, raws = build(tensors, **kw)
    want = plan_oracle.decode_plan(blob, state, out_len)
    n, got = dispatch(state, blob, out_len)
    assert n == sum(len(r) for r in raws)
    ts = P.decode_plan(state)
    for t, raw in zip(ts, raws):
        assert got[t.out_offset:t.out_offset + t.out_len] == raw
        assert want[t.out_offset:t.out_offset + t.out_len] == raw


ID, HUF, RANS, ILV = 0x0000, 0x0001, 0x0003, 0x7F01
NONE = (P.PLANE_OP_NONE, 0)


@pytest.mark.parametrize("elems", [1, 7, 16, 2047, 2048, 4097, 1 << 20, (1 << 22) + 33])
@pytest.mark.parametrize("codec", [HUF, ILV, ID])
def test_bf16_int_delta_exponent(elems, codec):
    note(f"bf16 IntDelta exponent elems={elems} codec={codec:#x}")
    raw = bf16_tensor(elems, elems, smooth=True)
    check([(P.CHAIN_IEEE16_SPLIT2, raw, [(ID, *NONE), (codec, P.PLANE_OP_INT_DELTA, 1)])])


@pytest.mark.parametrize("elems", [1, 5, 4096, 300001])
def test_fp32_predictor_xor_and_int_delta(elems):
    note(f"fp32 PredictorXor / IntDelta exponent elems={elems}")
    raw = fp32_tensor(elems, 3 + elems)
    check([(P.CHAIN_IEEE32_SPLIT4, raw, [(ID, *NONE), (HUF, *NONE), (HUF, *NONE), (HUF, P.PLANE_OP_PREDICTOR_XOR, 1)]),
           (P.CHAIN_IEEE32_SPLIT4, raw, [(ID, *NONE), (ID, *NONE), (HUF, *NONE), (RANS, P.PLANE_OP_INT_DELTA, 1)])])


@pytest.mark.parametrize("k", [1, 3, 4, 7])
def test_mantissa_zero_strip(k):
    note(f"MantissaZeroStrip k={k}")
    raw = fp32_tensor(100003, 40 + k, quant_bits=k)
    check([(P.CHAIN_IEEE32_SPLIT4, raw, [(HUF, P.PLANE_OP_MANTISSA_ZERO_STRIP, k), (ID, *NONE), (ID, *NONE), (HUF, *NONE)])])
    b = np.frombuffer(bf16_tensor(65536 + 3, k), np.uint16) & np.uint16(0xFFFF ^ ((1 << k) - 1))
    check([(P.CHAIN_IEEE16_SPLIT2, b.tobytes(), [(ILV, P.PLANE_OP_MANTISSA_ZERO_STRIP, k), (HUF, *NONE)])])


@pytest.mark.parametrize("width", [1, 2, 4, 8])
def test_passthrough_deltas_at_every_width(width):
    note(f"passthrough IntDelta / PredictorXor width={width}")
    rng = np.random.default_rng(width)
    raw = (np.cumsum(rng.integers(-3, 4, 123456 // width * width)) & 0xFF).astype(np.uint8).tobytes()
    check([(P.CHAIN_PASSTHROUGH, raw, [(HUF, P.PLANE_OP_INT_DELTA, width)])])
    if width <= 2:
        check([(P.CHAIN_PASSTHROUGH, raw[:65536], [(ID, P.PLANE_OP_PREDICTOR_XOR, width)])])


def test_many_tensors_with_ops_in_one_plan():
    note("40 tensors with ops in one plan")
    ts = []
    for i in range(40):
        raw = bf16_tensor(1000 + 977 * i, 100 + i, smooth=i % 2 == 0)
        op = [P.PLANE_OP_INT_DELTA, P.PLANE_OP_PREDICTOR_XOR, P.PLANE_OP_NONE][i % 3]
        ts.append((P.CHAIN_IEEE16_SPLIT2, raw, [(ID, *NONE), ([HUF, RANS, ILV][i % 3], op, 1 if op else 0)]))
    check(ts)


def test_crc_covers_the_decoded_plane_and_a_wrong_one_is_rejected():
    note("plane-op CRC semantics")
    raw = bf16_tensor(50000, 9, smooth=True)
    state, blob, out_len, _ = build([(P.CHAIN_IEEE16_SPLIT2, raw, [(ID, *NONE), (HUF, P.PLANE_OP_INT_DELTA, 1)])])
    assert dispatch(state, blob, out_len)[0] == len(raw)
    t = P.decode_plan(state)
    exp_plane = O.chain_forward(P.CHAIN_IEEE16_SPLIT2, raw)[1]
    # the CRC of the plane before the delta (the restored exponent plane) is wrong
    t[0].planes[1].crc32 = O.crc32(exp_plane)
    assert O.crc32(exp_plane) != O.crc32(O.int_delta(exp_plane))
    with pytest.raises(Exception) as ei:
        dispatch(P.encode_plan(t), blob, out_len)
    assert getattr(ei.value, "rc", None) == -1


def test_unsupported_and_invalid_ops():
    note("plane-op refusals")
    rng = np.random.default_rng(5)
    raw = rng.integers(0, 256, 4096, dtype=np.uint8).tobytes()
    state, blob, out_len, _ = build([(P.CHAIN_PASSTHROUGH, raw, [(ID, P.PLANE_OP_PREDICTOR_XOR, 4)])])
    with pytest.raises(Exception) as ei:  # PredictorXor at width 4: no LDS table on the device
        dispatch(state, blob, out_len)
    assert getattr(ei.value, "rc", None) == -5
    bad = bytearray(P.encode_plan([P.TensorPlan(P.CHAIN_E4M3_NIBBLE, 0, 16, [
        P.PlanePlan(ID, 0, 16, 16, None, None, P.PLANE_OP_INT_DELTA, 1),
        P.PlanePlan(ID, 0, 16, 16)])]))
    with pytest.raises(Exception) as ei:  # ops refuse nibble planes
        dispatch(bytes(bad), bytes(16), 16)
    assert getattr(ei.value, "rc", None) == -1
