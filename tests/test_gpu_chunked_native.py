"""Chunked GPU-native planes (huff_ilv / rans_ilv in chunk frames).

The reference frames every plane in chunks when a chunk size is set
(compressor.rs:316-381: per chunk [ver u8][state_len u32][state][payload],
with the plane's chunk table of (offset, decoded size)); the container reads
them per chunk (container.rs:1975-2050).  Each chunk payload here is this
library's own encoder output for that chunk's bytes; the plan decodes the
tensor bit-exactly through the fused route (chunk boundaries on 16384-symbol
blocks, same across planes: one sub-tensor per chunk, CRC partials
contiguous) or through plane scratch (other boundaries), and rejects a
native chunk that carries state.
"""
import sys
import time

import numpy as np
import pytest

import oracle as O
from ptwm_amd import api, ids, plan as P

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

LABEL = {"huff_ilv": ids.PLANE_CODEC_LABEL, "rans_ilv": ids.RANS_CODEC_LABEL}
WIRE = {"huff_ilv": ids.CODEC_HUFF_ILV, "rans_ilv": ids.CODEC_RANS_ILV}


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dev_bytes(b: bytes):
    t = torch.empty(max(1, len(b)), dtype=torch.uint8, device="cuda:0")
    if b:
        t[: len(b)].copy_(torch.from_numpy(np.frombuffer(b, np.uint8).copy()))
    return t[: len(b)]


def encode_plane(plane: bytes, codec: str) -> bytes:
    src = dev_bytes(plane)
    out = torch.empty(len(plane) * 2 + 65536, dtype=torch.uint8, device="cuda:0")
    n = api.plane_codec_encode_cuda(ids.PLANE_CODEC_LABEL, LABEL[codec], b"", src, out, 0)
    torch.cuda.synchronize()
    return out[:n].cpu().numpy().tobytes()


def framed(plane: bytes, codec: str, sizes, state=b""):
    """Chunk frames of `plane` cut at `sizes` -> (payload, chunk table)."""
    blob, ent, a = bytearray(), [], 0
    for sz in sizes:
        piece = plane[a:a + sz]
        pay = piece if codec == "identity" else encode_plane(piece, codec)
        ent.append((len(blob), sz))
        blob += b"\x00" + len(state).to_bytes(4, "little") + state + pay
        a += sz
    assert a == len(plane)
    return bytes(blob), ent


def cut(n, size):
    return [min(size, n - a) for a in range(0, n, size)]


def bf16(rows, cols, seed):
    w = (torch.randn(rows, cols, generator=torch.Generator().manual_seed(seed)) * 0.02).to(torch.bfloat16)
    return w.view(torch.uint8).reshape(-1).numpy().tobytes()


def run(tensors, data: bytes, out_len: int, reps: int = 1):
    """-> (bytes restored, output, best whole-call s, best decode-kernel ms)"""
    import ctypes as C
    from ptwm_amd._native import lib
    src = dev_bytes(data)
    out = torch.zeros(max(out_len, 1), dtype=torch.uint8, device="cuda:0")
    st = P.encode_plan(tensors)
    best, kbest = 1e9, 1e9
    ms = (C.c_float * 3)()
    lib().ptwm_mi355x_set_profiling(0, 1 if reps > 1 else 0)
    try:
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            n = api.hardware_backend_dispatch_decode_cuda(ids.HARDWARE_BACKEND_LABEL, ids.DECODE_PLAN_LABEL, st, src,
                                                          out, 0)
            torch.cuda.synchronize()
            best = min(best, time.perf_counter() - t0)
            if reps > 1:
                lib().ptwm_mi355x_last_kernel_ms(0, ms)
                kbest = min(kbest, ms[0])
    finally:
        lib().ptwm_mi355x_set_profiling(0, 0)
    return n, out.cpu().numpy().tobytes()[:out_len], best, kbest


def tensor_plan(data, chain, codecs, size, pad=0, crc=True):
    planes = O.chain_forward(chain, data)
    blob = bytearray(b"\x00" * pad)
    pps = []
    for pl, codec in zip(planes, codecs):
        pay, ent = framed(pl, codec, cut(len(pl), size))
        wire = 0 if codec == "identity" else WIRE[codec]
        pps.append(P.PlanePlan(wire, len(blob), len(pay), len(pl), ent, O.crc32(pl) if crc else None))
        blob += pay
        blob += b"\x00" * 3  # keep later payloads off 4-byte boundaries
    return P.TensorPlan(chain, 0, len(data), pps, xxh64=O.xxh64(data)), bytes(blob)


@pytest.mark.parametrize("codec", ["huff_ilv", "rans_ilv"])
def test_chunked_bf16_tensor_fused_route(codec):
    data = bf16(4096, 2048, 1)  # 16 MiB, 8 MiB planes
    t, blob = tensor_plan(data, P.CHAIN_IEEE16_SPLIT2, [codec, codec], 1 << 20, pad=5, crc=codec == "huff_ilv")
    n, got, _, _ = run([t], blob, len(data))  # CRC-32s (huff_ilv) and XXH64 checked
    assert n == len(data) and got == data
    t.xxh64 = None
    for p in t.planes:
        p.crc32 = None
    n, got, dt, kt = run([t], blob, len(data), reps=5)
    assert n == len(data) and got == data
    # the same tensor unchunked, for the rate
    planes = O.chain_forward(P.CHAIN_IEEE16_SPLIT2, data)
    pays = [encode_plane(pl, codec) for pl in planes]
    t2 = P.TensorPlan(P.CHAIN_IEEE16_SPLIT2, 0, len(data), [
        P.PlanePlan(WIRE[codec], 0, len(pays[0]), len(planes[0])),
        P.PlanePlan(WIRE[codec], len(pays[0]), len(pays[1]), len(planes[1]))])
    n2, got2, dt2, kt2 = run([t2], pays[0] + pays[1], len(data), reps=5)
    assert got2 == data
    note(f"{codec} 16 MiB bf16: chunked 1 MiB {dt * 1e3:.3f} ms call / {kt:.4f} ms decode kernel; "
         f"unchunked {dt2 * 1e3:.3f} ms call / {kt2:.4f} ms decode kernel")


def test_chunked_identity_and_native_planes_with_crc():
    data = bf16(1024, 3000, 2)
    t, blob = tensor_plan(data, P.CHAIN_IEEE16_SPLIT2, ["identity", "huff_ilv"], 1 << 18, pad=1)
    n, got, _, _ = run([t], blob, len(data))
    assert n == len(data) and got == data
    t.planes[1].crc32 ^= 1
    with pytest.raises(Exception) as ei:
        run([t], blob, len(data))
    assert getattr(ei.value, "rc", None) == -1


@pytest.mark.parametrize("chain", [P.CHAIN_E4M3_NIBBLE, P.CHAIN_PASSTHROUGH])
def test_chunked_planes_off_block_boundaries(chain):
    """Chunks of 100000 symbols (16-byte multiples, not 16384-symbol
    blocks): each chunk restores into plane scratch, then the merge."""
    x = np.random.default_rng(3).geometric(0.2, 1_234_560).clip(0, 255).astype(np.uint8)
    data = x.tobytes()
    t, blob = tensor_plan(data, chain, ["huff_ilv"] * P.CHAIN_PLANES[chain], 100_000, pad=2)
    n, got, _, _ = run([t], blob, len(data))
    assert n == len(data) and got == data


def test_native_chunk_with_state_is_invalid_and_unaligned_chunks_unsupported():
    x = np.random.default_rng(4).geometric(0.3, 200_000).clip(0, 255).astype(np.uint8).tobytes()
    pay, ent = framed(x, "huff_ilv", cut(len(x), 65536), state=b"\x01\x02")
    t = P.TensorPlan(P.CHAIN_PASSTHROUGH, 0, len(x), [P.PlanePlan(ids.CODEC_HUFF_ILV, 0, len(pay), len(x), ent)])
    with pytest.raises(Exception) as ei:
        run([t], pay, len(x))
    assert getattr(ei.value, "rc", None) == -1
    pay, ent = framed(x, "huff_ilv", cut(len(x), 1000))  # chunk offsets off 16-byte boundaries
    t = P.TensorPlan(P.CHAIN_PASSTHROUGH, 0, len(x), [P.PlanePlan(ids.CODEC_HUFF_ILV, 0, len(pay), len(x), ent)])
    with pytest.raises(Exception) as ei:
        run([t], pay, len(x))
    assert getattr(ei.value, "rc", None) == -5
