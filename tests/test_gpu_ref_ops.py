"""Encode-side plane ops and the chain trial on the device, against the oracle.

ptwm_mi355x_encode_tensor_ref_ops_cuda passes a plane through IntDelta,
PredictorXor or MantissaZeroStrip before its codec (the production split
chains with one plane op, python/ptwm/preprocessing/_chains.py:360-600), or
runs the reference's chain trial among those variants (compressor.rs:
504-640, restated as oracle.chain_trial: the smallest total payload wins,
the first on ties, a variant whose forward fails is skipped).  Payload bytes
and chosen variants equal the oracle's; the plans decode back on the device.
"""
import sys

import numpy as np
import pytest

import oracle as O
from ptwm_amd import api, ids, plan

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

HUF, RANS, ID, SEL = O.CODEC_HUFFMAN, O.CODEC_RANS, O.CODEC_IDENTITY, api.CODEC_SELECT
GPU_MENU = (HUF, RANS, ID)


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dev(b: bytes):
    t = torch.zeros(max(1, len(b)), dtype=torch.uint8, device="cuda:0")
    if b:
        t[: len(b)].copy_(torch.from_numpy(np.frombuffer(b, np.uint8).copy()))
    return t[: len(b)]


def host(t) -> bytes:
    torch.cuda.synchronize()
    return t.cpu().numpy().tobytes()


def bf16(n, seed, kind):
    g = torch.Generator().manual_seed(seed)
    if kind == "smooth":
        x = torch.cumsum(torch.randn(n, generator=g) * 0.01, 0) + torch.linspace(-3, 3, n)
    else:
        x = torch.randn(n, generator=g) * 0.02
    v = x.to(torch.bfloat16).view(torch.int16)
    if kind.startswith("q"):
        v = v & ~((1 << int(kind[1:])) - 1)
    return v.numpy().tobytes()


def fp32(n, seed, kind):
    g = torch.Generator().manual_seed(seed)
    x = torch.cumsum(torch.randn(n, generator=g) * 0.01, 0) if kind != "rand" else torch.randn(n, generator=g)
    v = x.to(torch.float32).view(torch.int32)
    if kind.startswith("q"):
        v = v & ~((1 << int(kind[1:])) - 1)
    return v.numpy().tobytes()


def encode(chain, data, codecs, ops, chunk=0, trial=False):
    out = torch.zeros(2 * len(data) + (1 << 20), dtype=torch.uint8, device="cuda:0")
    specs = None if ops is None else [api.plane_op_spec(o, p) for o, p in ops]
    used, st, chosen = api.encode_tensor_ref_ops_cuda(chain, codecs, specs, chunk, dev(data), out, 0, chain_trial=trial)
    return used, st, chosen, out


def decode_back(st, out, used, n):
    restored = torch.zeros(max(n, 1), dtype=torch.uint8, device="cuda:0")
    got = api.hardware_backend_dispatch_decode_cuda(ids.HARDWARE_BACKEND_LABEL, ids.DECODE_PLAN_LABEL, st,
                                                    out[:used], restored[:n], 0)
    return got, host(restored[:n])


EXPLICIT = [
    ("bf16-intdelta-huf", plan.CHAIN_IEEE16_SPLIT2, lambda: bf16(100003, 1, "smooth"), [HUF, HUF],
     [(0, 0), (O.PLANE_OP_INT_DELTA, 1)], 0),
    ("bf16-pxor-rans", plan.CHAIN_IEEE16_SPLIT2, lambda: bf16(70001, 2, "smooth"), [ID, RANS],
     [(0, 0), (O.PLANE_OP_PREDICTOR_XOR, 1)], 0),
    ("fp32-pxor-chunked", plan.CHAIN_IEEE32_SPLIT4, lambda: fp32(200000, 3, "smooth"), [HUF, HUF, HUF, HUF],
     [(0, 0), (0, 0), (0, 0), (O.PLANE_OP_PREDICTOR_XOR, 1)], 65536),
    ("fp32-mzs3", plan.CHAIN_IEEE32_SPLIT4, lambda: fp32(65537, 4, "q3"), [HUF, ID, ID, RANS],
     [(O.PLANE_OP_MANTISSA_ZERO_STRIP, 3), (0, 0), (0, 0), (O.PLANE_OP_INT_DELTA, 1)], 0),
    ("pass-intdelta-w2", plan.CHAIN_PASSTHROUGH, lambda: bf16(50000, 5, "smooth"), [HUF],
     [(O.PLANE_OP_INT_DELTA, 2)], 0),
    ("pass-pxor-w2", plan.CHAIN_PASSTHROUGH, lambda: bf16(30000, 6, "smooth"), [RANS],
     [(O.PLANE_OP_PREDICTOR_XOR, 2)], 0),
    ("pass-intdelta-w8", plan.CHAIN_PASSTHROUGH, lambda: fp32(40000, 7, "smooth"), [HUF],
     [(O.PLANE_OP_INT_DELTA, 8)], 4096),
]


@pytest.mark.parametrize("name,chain,make,codecs,ops,chunk", EXPLICIT, ids=[e[0] for e in EXPLICIT])
def test_explicit_plane_ops(name, chain, make, codecs, ops, chunk):
    note(f"encode with plane ops {name}")
    data = make()
    used, st, chosen, out = encode(chain, data, codecs, ops, chunk)
    assert chosen == [api.plane_op_spec(o, p) for o, p in ops]
    blob = host(out[:used])
    t = plan.decode_plan(st)[0]
    for p, (pp, (op, prm)) in enumerate(zip(t.planes, ops)):
        term = O.plane_op(op, prm, O.chain_forward(chain, data)[p], inverse=False)
        assert (pp.op, pp.op_param) == (op, prm), (name, p)
        payload = blob[pp.payload_offset: pp.payload_offset + pp.payload_len]
        if chunk:
            want, ent = O.encode_plane_chunked(codecs[p], term, chunk)
            assert [tuple(map(int, e)) for e in ent] == [tuple(c) for c in pp.chunks], (name, p)
        else:
            want = O.codec_encode(codecs[p], term)
        assert payload == want, (name, p)
    assert decode_back(st, out, used, len(data)) == (len(data), data)


def test_strip_refuses_a_plane_with_low_bits_set():
    note("MantissaZeroStrip refusal")
    data = fp32(4096, 8, "smooth")
    with pytest.raises(Exception) as ei:
        encode(plan.CHAIN_IEEE32_SPLIT4, data, [HUF] * 4, [(O.PLANE_OP_MANTISSA_ZERO_STRIP, 2), (0, 0), (0, 0), (0, 0)])
    assert getattr(ei.value, "rc", None) == -1


TRIAL = [
    ("bf16-random", plan.CHAIN_IEEE16_SPLIT2, lambda: bf16(131072, 11, "rand"), 0),
    ("bf16-smooth", plan.CHAIN_IEEE16_SPLIT2, lambda: bf16(131072, 12, "smooth"), 0),
    ("bf16-q4", plan.CHAIN_IEEE16_SPLIT2, lambda: bf16(131072, 13, "q4"), 0),
    ("bf16-q2-chunked", plan.CHAIN_IEEE16_SPLIT2, lambda: bf16(300000, 14, "q2"), 65536),
    ("fp32-smooth", plan.CHAIN_IEEE32_SPLIT4, lambda: fp32(65536, 15, "smooth"), 0),
    ("fp32-q1", plan.CHAIN_IEEE32_SPLIT4, lambda: fp32(65536, 16, "q1"), 0),
]


@pytest.mark.parametrize("name,chain,make,chunk", TRIAL, ids=[t[0] for t in TRIAL])
def test_chain_trial_matches_the_oracle(name, chain, make, chunk):
    note(f"chain trial {name}")
    data = make()
    np_ = plan.CHAIN_PLANES[chain]
    used, st, chosen, out = encode(chain, data, [SEL] * np_, None, chunk, trial=True)
    want_ops, want_enc = O.chain_trial(chain, data, GPU_MENU)
    assert chosen == [api.plane_op_spec(o, p) for o, p in want_ops], (name, chosen, want_ops)
    blob = host(out[:used])
    t = plan.decode_plan(st)[0]
    planes = O.chain_forward(chain, data)
    for p, pp in enumerate(t.planes):
        codec, whole = want_enc[p]
        assert pp.codec == codec and (pp.op, pp.op_param) == want_ops[p], (name, p)
        payload = blob[pp.payload_offset: pp.payload_offset + pp.payload_len]
        if chunk:
            term = O.plane_op(*want_ops[p], planes[p], inverse=False)
            want, ent = O.encode_plane_chunked(codec, term, chunk)
            assert [tuple(map(int, e)) for e in ent] == [tuple(c) for c in pp.chunks], (name, p)
        else:
            want = whole
        assert payload == want, (name, p)
    assert decode_back(st, out, used, len(data)) == (len(data), data)


def test_chain_trial_ties_go_to_the_first_variant():
    """Identity payloads are the planes themselves: every variant that runs
    has the same total, so the plain split (first in the list) wins."""
    note("chain trial tie")
    data = bf16(20000, 17, "q4")
    used, st, chosen, out = encode(plan.CHAIN_IEEE16_SPLIT2, data, [ID, ID], None, 0, trial=True)
    assert chosen == [0, 0]
    assert O.chain_trial(plan.CHAIN_IEEE16_SPLIT2, data, (ID,))[0] == [(0, 0), (0, 0)]
