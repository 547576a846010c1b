"""GPU parity of the packed-nibble payload form (tag 2) of both GPU-native
plane codecs (huff_ilv and rans_ilv):

- GPU encode of near-uniform nibble planes gives the specification's bytes
  ([2][n u32][0 0 0][byte i = s[2i] | s[2i+1] << 4], oracle encoders);
- the fused decoders restore packed payloads (even and odd n, partial last
  block and group) and reject malformed ones where the specification's
  decoder does;
- tensor level: an MXFP4 tensor (nibble split) whose planes are packed goes
  through GPU encode -> fused decode -> merge bit-exact;
- a coded payload that happens to have the stored or packed length (the
  host reserves LDS tables only for planes of other lengths) decodes through
  the kernel's retry with a table for every plane.
"""
import sys

import numpy as np
import pytest

import oracle as O
from ptwm_amd import api, ids, plan

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

SEL = ids.PLANE_CODEC_LABEL
CODECS = [
    ("huff_ilv", ids.PLANE_CODEC_LABEL, O.ilv_encode, O.ilv_decode, ids.CODEC_HUFF_ILV),
    ("rans_ilv", ids.RANS_CODEC_LABEL, O.rans_ilv_encode, O.rans_ilv_decode, ids.CODEC_RANS_ILV),
]
SIZES = (16, 17, 18, 31, 1001, 16384, 16385, 3 * 16384 + 77, 200_001)


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dev(b: bytes):
    a = np.frombuffer(bytes(b), np.uint8)
    t = torch.zeros(max(len(a), 1), dtype=torch.uint8, device="cuda:0")
    if len(a):
        t[: len(a)].copy_(torch.from_numpy(a.copy()))
    return t[: len(a)]


def host(t) -> bytes:
    torch.cuda.synchronize()
    return t.cpu().numpy().tobytes()


def gpu_encode(label, src: bytes) -> bytes:
    out = torch.zeros(len(src) + 1, dtype=torch.uint8, device="cuda:0")
    n = api.plane_codec_encode_cuda(SEL, label, b"", dev(src), out, 0)
    return host(out)[:n]


def gpu_decode(label, payload: bytes, cap: int):
    dst = torch.zeros(max(cap, 1), dtype=torch.uint8, device="cuda:0")[:cap]
    try:
        n = api.plane_codec_decode_cuda(SEL, label, b"", dev(payload), dst, 0)
    except Exception as e:  # noqa: BLE001
        return getattr(e, "rc", -99), None
    return n, host(dst)[:n]


@pytest.mark.parametrize("name,label,enc,dec,wire", CODECS, ids=[c[0] for c in CODECS])
def test_packed_encode_decode_matches_spec(name, label, enc, dec, wire):
    rng = np.random.default_rng(21)
    for n in SIZES:
        src = rng.integers(0, 16, n).astype(np.uint8).tobytes()
        note(f"{name} packed n={n}")
        want = enc(src)
        assert want[0] == 2, n                      # the specification picks packed here
        assert gpu_encode(label, src) == want, n
        got_n, got = gpu_decode(label, want, n)
        assert got_n == n and got == src, n


@pytest.mark.parametrize("name,label,enc,dec,wire", CODECS, ids=[c[0] for c in CODECS])
def test_packed_malformed_matches_spec(name, label, enc, dec, wire):
    rng = np.random.default_rng(22)
    for n in (101, 16385):
        good = bytearray(enc(rng.integers(0, 16, n).astype(np.uint8).tobytes()))
        variants = [
            bytes(good[:-1]),                                   # truncated
            bytes(good) + b"\0",                                # one byte too many
            bytes(good[:5]) + b"\1" + bytes(good[6:]),          # pad byte set
            bytes(good[:7]) + b"\x80" + bytes(good[8:]),        # pad byte set
            bytes(good[:1]) + (n + 2).to_bytes(4, "little") + bytes(good[5:]),  # length mismatch
            bytes(good[:1]) + (n - 1).to_bytes(4, "little") + bytes(good[5:]),
            bytes(good[:7]),                                    # header only, short
        ]
        if n & 1:
            variants.append(bytes(good[:-1]) + bytes([good[-1] | 0x10]))   # high nibble past n
        for k, b in enumerate(variants):
            note(f"{name} packed malformed n={n} variant={k}")
            try:
                want = dec(b, n)
            except O.OracleError:
                want = None
            got_n, got = gpu_decode(label, b, n)
            if want is None:
                assert got_n < 0, (n, k)
            else:
                assert got_n == len(want) and got == want, (n, k)


@pytest.mark.parametrize("name,label,enc,dec,wire", CODECS, ids=[c[0] for c in CODECS])
def test_mxfp4_tensor_with_packed_planes(name, label, enc, dec, wire):
    note(f"{name} mxfp4 tensor")
    for n in (123_457, 1 << 20):
        data = np.random.default_rng(n).integers(0, 256, n).astype(np.uint8).tobytes()
        out = torch.zeros(n * 2 + 65536, dtype=torch.uint8, device="cuda:0")
        used, st = api.encode_tensor_cuda(plan.CHAIN_NIBBLE_SPLIT, dev(data), out, 0, codec=name)
        t = plan.decode_plan(st)[0]
        blob = host(out[:used])
        planes = O.chain_forward(plan.CHAIN_NIBBLE_SPLIT, data)
        for p, want in zip(t.planes, planes):
            payload = blob[p.payload_offset: p.payload_offset + p.payload_len]
            assert p.codec == wire and payload[0] == 2 and payload == enc(want), n
        restored = torch.zeros(n, dtype=torch.uint8, device="cuda:0")
        got = api.hardware_backend_dispatch_decode_cuda(ids.HARDWARE_BACKEND_LABEL, ids.DECODE_PLAN_LABEL, st,
                                                        out[:used], restored, 0)
        assert got == n and host(restored) == data


def _collision(enc, target, ns, gen):
    """First n (deterministic per-n data) whose coded payload has length
    target(n)."""
    for n in ns:
        x = gen(np.random.default_rng(n), n)
        c = enc(x)
        if len(c) == target(n):
            return x, c
    raise AssertionError("no length collision found")


def _skewed_bytes(rng, n):
    return np.minimum(rng.geometric(0.004, n), 255).astype(np.uint8).tobytes()


def _skewed_nibbles(rng, n):
    x = (rng.integers(0, 16, n) & rng.integers(0, 16, n)) | rng.integers(0, 2, n)
    return (x & 15).astype(np.uint8).tobytes()


COLLISIONS = [
    ("huff_ilv-stored-length", ids.PLANE_CODEC_LABEL, O.ilv_encode_coded, ids.CODEC_HUFF_ILV,
     lambda n: n + 1, range(1000, 40000), _skewed_bytes),
    ("huff_ilv-packed-length", ids.PLANE_CODEC_LABEL, O.ilv_encode_coded, ids.CODEC_HUFF_ILV,
     lambda n: 8 + (n + 1) // 2, range(2000, 60000), _skewed_nibbles),
    ("rans_ilv-stored-length", ids.RANS_CODEC_LABEL, O.rans_ilv_encode_coded, ids.CODEC_RANS_ILV,
     lambda n: n + 1, range(1000, 40000), _skewed_bytes),
]


@pytest.mark.parametrize("name,label,enc,wire,target,ns,gen", COLLISIONS, ids=[c[0] for c in COLLISIONS])
def test_coded_payload_with_stored_or_packed_length(name, label, enc, wire, target, ns, gen):
    """A coded (tag 1) payload whose length equals the stored (n + 1) or the
    packed (8 + ceil(n / 2)) length: the host reserves no LDS table for a
    plane of those lengths, the kernel reports it, and the tensor is decoded
    again with a table for every plane.  Plane level, then a two-plane bf16
    tensor whose other plane is coded too (slot numbering)."""
    x, payload = _collision(enc, target, ns, gen)
    n = len(x)
    assert payload[0] == 1
    note(f"{name} n={n}")
    got_n, got = gpu_decode(label, payload, n)
    assert got_n == n and got == x
    # tensor level: plane 0 the colliding payload, plane 1 an ordinary coded one
    other = np.minimum(np.random.default_rng(99).geometric(0.3, n), 255).astype(np.uint8).tobytes()
    p1 = enc(other)
    assert p1[0] == 1 and len(p1) not in (n + 1, 8 + (n + 1) // 2)
    blob = bytearray(payload)
    off1 = (len(blob) + 255) // 256 * 256
    blob += b"\0" * (off1 - len(blob)) + p1
    pl = [plan.PlanePlan(wire, 0, len(payload), n), plan.PlanePlan(wire, off1, len(p1), n)]
    data = O.chain_inverse(O.CHAIN_IEEE16_SPLIT2, [x, other])
    st = plan.encode_plan([plan.TensorPlan(plan.CHAIN_IEEE16_SPLIT2, 0, len(data), pl)])
    restored = torch.zeros(len(data), dtype=torch.uint8, device="cuda:0")
    got = api.hardware_backend_dispatch_decode_cuda(ids.HARDWARE_BACKEND_LABEL, ids.DECODE_PLAN_LABEL, st,
                                                    dev(bytes(blob)), restored, 0)
    assert got == len(data) and host(restored) == data
