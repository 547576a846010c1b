"""Parallel decode of reference Huffman payloads (decode_sync.hip) against
the CPU oracle (the reference decoder, decompress.rs:8-211).

Payloads of at least 16 KiB take the parallel path; it must restore exactly
the oracle's bytes, and a payload it declines (malformed, trailing bytes)
must still get the oracle's outcome through the exact path.  Each case is
decoded through the plane-level device entry point.
"""
import struct
import sys

import numpy as np
import pytest

import oracle as O
from ptwm_amd import api, ids

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

SEL = ids.PLANE_CODEC_LABEL


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dev(b: bytes):
    t = torch.zeros(len(b) + 16, dtype=torch.uint8, device="cuda:0")
    if b:
        t[: len(b)].copy_(torch.from_numpy(np.frombuffer(b, np.uint8).copy()))
    return t[: len(b)]


def gpu_decode(payload: bytes, cap: int):
    out = torch.zeros(cap + 16, dtype=torch.uint8, device="cuda:0")
    try:
        n = api.plane_codec_decode_cuda(SEL, "huffman", b"", dev(payload), out[:cap], 0)
    except Exception as e:  # noqa: BLE001
        return None, getattr(e, "rc", None)
    torch.cuda.synchronize()
    return out[:n].cpu().numpy().tobytes(), n


def oracle_decode(payload: bytes, cap: int):
    try:
        return O.codec_decode(O.CODEC_HUFFMAN, payload, cap)
    except Exception:  # noqa: BLE001
        return None


def planes():
    rng = np.random.default_rng(23)
    yield "geo100k", rng.geometric(0.3, 100_000).clip(0, 255).astype(np.uint8).tobytes()
    w = (torch.randn(1 << 20, generator=torch.Generator().manual_seed(2)) * 0.02).to(torch.bfloat16)
    yield "bf16exp1m", O.chain_forward(O.CHAIN_IEEE16_SPLIT2, w.view(torch.uint8).numpy().tobytes())[1]
    yield "bf16mant1m", O.chain_forward(O.CHAIN_IEEE16_SPLIT2, w.view(torch.uint8).numpy().tobytes())[0]
    # 1-bit codes: more symbols per wavefront than the LDS output stage holds
    yield "two2m", rng.choice([3, 9], 2 << 20, p=[0.97, 0.03]).astype(np.uint8).tobytes()
    yield "uni16", rng.integers(0, 16, 300_000).astype(np.uint8).tobytes()
    f = [1, 1]
    while len(f) < 20:
        f.append(f[-1] + f[-2])
    p = np.array(f, float)
    yield "fib11bit", rng.choice(20, 500_000, p=p / p.sum()).astype(np.uint8).tobytes()
    x = torch.randn(2048, 4096, generator=torch.Generator().manual_seed(3))
    x = (x / x.abs().amax(1, keepdim=True) * 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy().tobytes()
    hi, lo = O.chain_forward(O.CHAIN_E4M3_NIBBLE, x)
    yield "e4m3hi8m", hi
    yield "e4m3lo8m", lo


@pytest.mark.parametrize("name,plane", list(planes()), ids=[n for n, _ in planes()])
def test_parallel_huffman_decode_matches_reference(name, plane):
    payload = O.codec_encode(O.CODEC_HUFFMAN, plane)
    note(f"sync decode {name}: plane {len(plane)} payload {len(payload)} tag {payload[0]}")
    before = api.decode_stats(0)
    got, n = gpu_decode(payload, len(plane))
    assert n == len(plane) and got == plane
    after = api.decode_stats(0)
    if payload[0] == 1 and len(payload) >= 16384:  # a coded payload on the parallel path: accepted there
        assert after["accepted"] == before["accepted"] + 1 and after["fallbacks"] == before["fallbacks"], after


def _streams_start(payload: bytes) -> int:
    blob = payload[5:]
    _, used = O.huf_decode_weights(blob)
    return 5 + used + 16


def _fixed_length_code(payload: bytes) -> bool:
    lengths = [w for w in O.huf_decode_weights(payload[5:])[0] if w]
    return len(set(lengths)) == 1


@pytest.mark.parametrize("kind", ["geometric", "uniform16"])
def test_parallel_huffman_malformed_matches_reference_outcome(kind):
    """Malformed payloads of a variable-length code, and of a fixed-length one
    (16 near-equiprobable symbols: every code 4 bits, whose codeword starts
    the parallel path computes instead of finding), decode or fail exactly as
    the reference decoder."""
    rng = np.random.default_rng(99)
    if kind == "geometric":
        base = rng.geometric(0.25, 200_000).clip(0, 255).astype(np.uint8).tobytes()
    else:
        base = rng.integers(0, 16, 200_000).astype(np.uint8).tobytes()
    payload = O.codec_encode(O.CODEC_HUFFMAN, base)
    assert payload[0] == 1 and _fixed_length_code(payload) == (kind == "uniform16")
    s0 = _streams_start(payload)
    jump = struct.unpack_from("<4I", payload, s0 - 16)
    cases = []
    for k in range(30):                                   # bit flips inside the streams
        b = bytearray(payload)
        for _ in range(1 + k % 3):
            i = int(rng.integers(s0, len(b)))
            b[i] ^= 1 << int(rng.integers(0, 8))
        cases.append((f"flip{k}", bytes(b)))
    for s in range(4):                                    # first byte of each stream (the end bits)
        b = bytearray(payload)
        b[s0 + sum(jump[:s])] ^= 0x80
        cases.append((f"lastbits{s}", bytes(b)))
    b = bytearray(payload)                                # a zero byte appended to stream 3
    b += b"\x00"
    struct.pack_into("<I", b, s0 - 4, jump[3] + 1)
    cases.append(("trailing0", bytes(b)))
    b = bytearray(payload)                                # streams 0/1 boundary moved by one byte
    struct.pack_into("<I", b, s0 - 16, jump[0] + 1)
    struct.pack_into("<I", b, s0 - 12, jump[1] - 1)
    cases.append(("moved", bytes(b)))
    cases.append(("truncated", payload[:-7]))
    for name, p in cases:
        note(f"sync malformed {name}")
        want = oracle_decode(p, len(base))
        got, _ = gpu_decode(p, len(base))
        assert (got is None) == (want is None), name
        if want is not None:
            assert got == want, name


def test_unsettled_streams_take_the_host_fix_passes(monkeypatch):
    """A stream the queued fix passes leave unsettled gets more passes from
    the host, then its offsets, write and verdict again.  The library's test
    mode (PTWM_SYNC_FORCE_UNSETTLED) drops the first pass's look-back and
    marks every stream its queued fix pass touches, so this path runs."""
    rng = np.random.default_rng(5)
    plane = rng.geometric(0.3, 300_000).clip(0, 255).astype(np.uint8).tobytes()
    payload = O.codec_encode(O.CODEC_HUFFMAN, plane)
    bad = bytearray(payload)
    bad[len(bad) // 2] ^= 0x10
    bad = bytes(bad)
    monkeypatch.setenv("PTWM_SYNC_FORCE_UNSETTLED", "1")
    note("sync forced-unsettled: valid payload")
    before = api.decode_stats(0)
    got, n = gpu_decode(payload, len(plane))
    after = api.decode_stats(0)
    assert n == len(plane) and got == plane
    assert after["extra_rounds"] == before["extra_rounds"] + 1, after
    assert after["accepted"] == before["accepted"] + 1, after
    note("sync forced-unsettled: one bit flipped")
    want = oracle_decode(bad, len(plane))
    got, _ = gpu_decode(bad, len(plane))
    assert (got is None) == (want is None) and (want is None or got == want)


def _random_plane(rng, n):
    kind = int(rng.integers(0, 6))
    if kind == 0:
        return rng.geometric(float(rng.choice([0.05, 0.2, 0.5, 0.8])), n).clip(0, 255).astype(np.uint8)
    if kind == 1:  # uniform over k symbols (16: a fixed-length code; 256: stored)
        return rng.integers(0, int(rng.choice([2, 3, 16, 64, 256])), n).astype(np.uint8)
    if kind == 2:  # Zipf-like
        return (rng.zipf(float(rng.choice([1.3, 2.0])), n) % 256).astype(np.uint8)
    if kind == 3:  # two clusters
        return np.where(rng.random(n) < 0.7, rng.integers(100, 104, n), rng.integers(0, 256, n)).astype(np.uint8)
    if kind == 4:  # runs
        return np.repeat(rng.integers(0, 8, n // 64 + 1), 64)[:n].astype(np.uint8)
    return (rng.normal(128, float(rng.choice([1.0, 6.0, 30.0])), n).clip(0, 255)).astype(np.uint8)


@pytest.mark.parametrize("seed", range(10))
def test_parallel_huffman_batches_match_reference(seed):
    """Several reference Huffman payloads of varied sizes and symbol
    distributions in one launch (passthrough tensors of one plan): their
    subsequence sizes, fixed- and variable-length codes and stored payloads
    mix in the passes; every tensor restores the oracle decoder's bytes.  In
    half the batches one payload has a stream bit flipped, and the call then
    fails exactly when the oracle decoder rejects that payload."""
    from ptwm_amd import plan as P
    rng = np.random.default_rng(1000 + seed)
    k = int(rng.integers(2, 7))
    planes = [_random_plane(rng, int(rng.integers(20_000, 2_500_000))).tobytes() for _ in range(k)]
    payloads = [O.codec_encode(O.CODEC_HUFFMAN, pl) for pl in planes]
    bad = int(rng.integers(0, k)) if seed % 2 else -1
    if bad >= 0 and payloads[bad][0] == 1:
        b = bytearray(payloads[bad])
        i = int(rng.integers(_streams_start(payloads[bad]), len(b)))
        b[i] ^= 1 << int(rng.integers(0, 8))
        payloads[bad] = bytes(b)
    blob, tensors, off_out = b"", [], 0
    for pl, pay in zip(planes, payloads):
        tensors.append(P.TensorPlan(P.CHAIN_PASSTHROUGH, off_out, len(pl),
                                    [P.PlanePlan(O.CODEC_HUFFMAN, len(blob), len(pay), len(pl))]))
        blob += pay + bytes(-len(pay) % 16)
        off_out += (len(pl) + 255) // 256 * 256
    want = [oracle_decode(pay, len(pl)) for pl, pay in zip(planes, payloads)]
    note(f"sync batch {seed}: {k} payloads, sizes {[len(p) for p in planes]}, tags {[p[0] for p in payloads]}, "
         f"corrupted {bad}, oracle rejects {[w is None for w in want]}")
    out = torch.zeros(off_out + 16, dtype=torch.uint8, device="cuda:0")
    try:
        n = api.hardware_backend_dispatch_decode_cuda(ids.HARDWARE_BACKEND_LABEL, ids.DECODE_PLAN_LABEL,
                                                      P.encode_plan(tensors), dev(blob), out[:off_out], 0)
        torch.cuda.synchronize()
    except Exception:  # noqa: BLE001
        n = None
    assert (n is None) == any(w is None for w in want)
    if n is not None:
        got = out.cpu().numpy().tobytes()
        for t, w in zip(tensors, want):
            assert got[t.out_offset:t.out_offset + t.out_len] == w


@pytest.mark.parametrize("n", [4095, 4096, 4097, 65536, 65539, (1 << 20) + 1, 3 * (1 << 20) + 7])
def test_stored_payload_copy(n):
    """Stored (tag 0) payloads of 4 KiB and more are copied by the
    multi-workgroup copy kernel; the source sits one byte past the tag."""
    plane = np.random.default_rng(n).integers(0, 256, n, dtype=np.uint8).tobytes()
    for codec, name in [(O.CODEC_HUFFMAN, "huffman"), (O.CODEC_RANS, "rans")]:
        payload = O.codec_encode(codec, plane)
        assert payload[0] == 0
        note(f"stored copy {name} n={n}")
        out = torch.zeros(n + 16, dtype=torch.uint8, device="cuda:0")
        got = api.plane_codec_decode_cuda(SEL, name, b"", dev(payload), out[:n], 0)
        torch.cuda.synchronize()
        assert got == n and out[:n].cpu().numpy().tobytes() == plane
