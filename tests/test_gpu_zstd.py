"""Zstd payloads (codec 0x0004) decoded on the device against the oracle.

Frames written by the image's libzstd (tests/zstd_frames.py: every level,
checksums, content sizes, windows, concatenated and skippable frames) go
through decode plans, whole and in chunk frames at odd offsets, and must
come back bit-exact; malformed ones must be InvalidInput (-1) exactly where
the oracle's RFC 8878 restatement (pinned by libzstd and by the reference's
fixture planes on CPU) rejects them.  The reference's own Zstd planes are
decoded on the device by test_gpu_container.py.
"""
import sys

import numpy as np
import pytest

import oracle as O
from ptwm_amd import api, ids, plan as P

import zstd_frames as ZF

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

SAMPLES = list(ZF.samples())


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dev_bytes(b: bytes):
    t = torch.empty(max(1, len(b)), dtype=torch.uint8, device="cuda:0")
    if b:
        t[: len(b)].copy_(torch.from_numpy(np.frombuffer(b, np.uint8).copy()))
    return t[: len(b)]


def dispatch(tensors, data: bytes, out_len: int):
    src = dev_bytes(data)
    out = torch.full((max(out_len, 1),), 0x5A, dtype=torch.uint8, device="cuda:0")
    n = api.hardware_backend_dispatch_decode_cuda(ids.HARDWARE_BACKEND_LABEL, ids.DECODE_PLAN_LABEL,
                                                  P.encode_plan(tensors), src, out, 0)
    torch.cuda.synchronize()
    return n, out.cpu().numpy().tobytes()[:out_len]


def one(payload: bytes, n: int, chunks=None):
    return [P.TensorPlan(P.CHAIN_PASSTHROUGH, 0, n, [P.PlanePlan(O.CODEC_ZSTD, 0, len(payload), n, chunks)])]


@pytest.mark.parametrize("name,data", SAMPLES, ids=[n for n, _ in SAMPLES])
@pytest.mark.parametrize("level", [-5, 1, 3, 19])
def test_zstd_frames_decode_on_device(name, data, level):
    if not data:
        pytest.skip("an empty plane has no payload bytes to plan")
    note(f"zstd {name} level={level} n={len(data)}")
    f = ZF.compress(data, level)
    assert O.zstd_decompress(f, len(data)) == data
    n, got = dispatch(one(f, len(data)), f, len(data))
    assert n == len(data) and got == data


def test_frame_options_and_multi_frame_payloads():
    data = SAMPLES[0][1]
    cases = [ZF.compress(data, 3, checksum=True), ZF.compress(data, 1, content_size=False),
             ZF.compress(data, 19, window_log=10), ZF.compress(data, 3, checksum=True, content_size=False)]
    a, b = data[:40_000], SAMPLES[2][1][:90_000]
    cases.append(ZF.skippable(b"x" * 17) + ZF.compress(a, 3) + ZF.skippable(b"", 3) + ZF.compress(b, 9, checksum=True))
    wants = [data] * 4 + [a + b]
    for k, (f, want) in enumerate(zip(cases, wants)):
        note(f"zstd option case {k}")
        n, got = dispatch(one(f, len(want)), f, len(want))
        assert n == len(want) and got == want, k


def test_chunked_zstd_planes_of_a_bf16_tensor():
    w = (torch.randn(1500, 1000, generator=torch.Generator().manual_seed(4)) * 0.02).to(torch.bfloat16)
    data = w.view(torch.uint8).reshape(-1).numpy().tobytes()
    planes = O.chain_forward(P.CHAIN_IEEE16_SPLIT2, data)
    # chunk frames [ver][state_len][payload] of 256 KiB, as compressor.rs:316-381 writes them
    blob = bytearray(b"\x00" * 3)
    pp = []
    for pl in planes:
        start = len(blob)
        ent = []
        for k in range(0, len(pl), 1 << 18):
            c = ZF.compress(pl[k:k + (1 << 18)], 3)
            ent.append((len(blob) - start, min(1 << 18, len(pl) - k)))
            blob += b"\x00" + b"\x00\x00\x00\x00" + c
        pp.append(P.PlanePlan(O.CODEC_ZSTD, start, len(blob) - start, len(pl), ent, crc32=O.crc32(pl)))
    t = P.TensorPlan(P.CHAIN_IEEE16_SPLIT2, 0, len(data), pp, xxh64=O.xxh64(data))
    n, got = dispatch([t], bytes(blob), len(data))
    assert n == len(data) and got == data


def test_corruptions_rejected_where_the_oracle_rejects():
    data = SAMPLES[2][1][:120_000]
    f = ZF.compress(data, 3, checksum=True)
    rng = np.random.default_rng(7)
    bad = [f[:-1], f[: len(f) // 2], f + b"\x00", bytes([f[0] ^ 1]) + f[1:]]
    for _ in range(12):
        b = bytearray(f)
        b[int(rng.integers(8, len(b) - 4))] ^= int(rng.integers(1, 256))
        bad.append(bytes(b))
    for k, b in enumerate(bad):
        try:
            want = O.zstd_decompress(b, len(data))
            oracle_ok = len(want) == len(data)
        except O.OracleError:
            oracle_ok = False
        note(f"zstd corruption {k}: oracle {'accepts' if oracle_ok else 'rejects'}")
        try:
            n, got = dispatch(one(b, len(data)), b, len(data))
            dev_ok = True
        except Exception as e:
            assert getattr(e, "rc", None) == -1, k
            dev_ok = False
        assert dev_ok == oracle_ok, k
        if dev_ok:
            assert got == want
    # the plan's length disagrees with the frame's: InvalidInput
    with pytest.raises(Exception) as ei:
        dispatch(one(f, len(data) + 1), f, len(data) + 1)
    assert getattr(ei.value, "rc", None) == -1


@pytest.mark.parametrize("period", [8 * 1024 + 3, 40 * 1024 + 1, 200 * 1024 + 7])
def test_matches_beyond_the_history_ring(period):
    """Random bytes repeated with a period past the decoder's 8 KiB LDS
    history ring: every match reads the plane itself, often bytes the same
    sequence batch stored (the decoder fences before reading bytes stored
    since its last fence), and with the 200 KiB period across blocks."""
    rng = np.random.default_rng(period)
    unit = rng.integers(0, 256, period, dtype=np.uint8).tobytes()
    data = (unit * (3 + (600 * 1024) // period))[:600 * 1024 + 11]
    for level in (1, 9):
        note(f"zstd repeat period {period} level {level}")
        f = ZF.compress(data, level, window_log=20)
        assert O.zstd_decompress(f, len(data)) == data
        n, got = dispatch(one(f, len(data)), f, len(data))
        assert n == len(data) and got == data
