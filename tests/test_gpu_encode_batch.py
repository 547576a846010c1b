"""GPU batched tensor encode (ptwm_mi355x_encode_tensors_cuda): many
tensors of several chains and sizes in one call.

- every plane payload equals the one the single-tensor encoder writes for
  that tensor (which the per-codec tests pin to the format specification);
- the returned plan restores every tensor bit-exact through the
  tensor-level decode entry point;
- a too-small output buffer reports BufferTooSmall with a sufficient size.
"""
import sys

import numpy as np
import pytest

from ptwm_amd import api, ids, plan

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def host(t) -> bytes:
    torch.cuda.synchronize()
    return t.cpu().numpy().tobytes()


def tensors():
    g = torch.Generator(device="cuda:0").manual_seed(5)
    out = [
        (plan.CHAIN_IEEE16_SPLIT2, (torch.randn(3 << 20, generator=g, device="cuda:0") * 0.02).to(torch.bfloat16)),
        (plan.CHAIN_IEEE16_SPLIT2, (1 + 0.01 * torch.rand(4096, generator=g, device="cuda:0")).to(torch.bfloat16)),
        (plan.CHAIN_IEEE32_SPLIT4, torch.randn(100_003, generator=g, device="cuda:0") * 0.02),
        (plan.CHAIN_E4M3_NIBBLE, (torch.randn(1 << 20, generator=g, device="cuda:0") * 50).clamp(-448, 448)
         .to(torch.float8_e4m3fn)),
        (plan.CHAIN_NIBBLE_SPLIT, torch.randint(0, 256, (77_777,), generator=g, device="cuda:0", dtype=torch.uint8)),
        (plan.CHAIN_PASSTHROUGH, torch.randint(120, 128, (5000,), generator=g, device="cuda:0", dtype=torch.uint8)),
        (plan.CHAIN_IEEE16_SPLIT2, torch.zeros(0, device="cuda:0", dtype=torch.bfloat16)),
    ]
    return [(c, t.contiguous().view(torch.uint8)) for c, t in out]


@pytest.mark.parametrize("codec", ["huff_ilv", "rans_ilv"])
def test_batch_encode_matches_single_and_round_trips(codec):
    items = tensors()
    total = sum(t.numel() for _, t in items)
    out = torch.zeros(total * 2 + (1 << 20), dtype=torch.uint8, device="cuda:0")
    note(f"batch encode {codec}: {len(items)} tensors, {total} bytes")
    used, st = api.encode_tensors_cuda(items, out, 0, codec=codec)
    blob = host(out[:used])
    tp = plan.decode_plan(st)
    assert len(tp) == len(items)
    off = 0
    for (chain, src), t in zip(items, tp):
        assert t.chain == chain and t.out_len == src.numel() and t.out_offset == off
        off = (off + src.numel() + 255) // 256 * 256
        one = torch.zeros(src.numel() * 2 + 65536, dtype=torch.uint8, device="cuda:0")
        u1, s1 = api.encode_tensor_cuda(chain, src, one, 0, codec=codec)
        b1 = host(one[:u1])
        for p, q in zip(t.planes, plan.decode_plan(s1)[0].planes):
            assert p.codec == q.codec and p.plane_len == q.plane_len
            assert blob[p.payload_offset: p.payload_offset + p.payload_len] == \
                b1[q.payload_offset: q.payload_offset + q.payload_len]
    restored = torch.zeros(max(off, 1), dtype=torch.uint8, device="cuda:0")
    n = api.hardware_backend_dispatch_decode_cuda(ids.HARDWARE_BACKEND_LABEL, ids.DECODE_PLAN_LABEL, st,
                                                  out[:used], restored, 0)
    assert n == total
    r = host(restored)
    for (chain, src), t in zip(items, tp):
        assert r[t.out_offset: t.out_offset + t.out_len] == host(src)


@pytest.mark.parametrize("codec", ["huff_ilv", "rans_ilv"])
def test_batch_encode_many_small_batches(codec):
    """With the batch size set below the tensors' sizes, one call runs one
    batch per tensor or two: payload offsets of later batches (the per-batch
    base), the plan and the round trip must be the same as with one batch;
    and when the output runs out in the second batch, the reported size is
    enough."""
    from ptwm_amd._native import lib

    items = tensors()
    total = sum(t.numel() for _, t in items)
    out1 = torch.zeros(total * 2 + (1 << 20), dtype=torch.uint8, device="cuda:0")
    used1, st1 = api.encode_tensors_cuda(items, out1, 0, codec=codec)
    L = lib()
    try:
        assert L.ptwm_mi355x_set_encode_batch_bytes(1 << 20, 0) == 0
        out = torch.zeros(total * 2 + (1 << 20), dtype=torch.uint8, device="cuda:0")
        note(f"batch encode {codec} in 1 MiB batches")
        used, st = api.encode_tensors_cuda(items, out, 0, codec=codec)
        b1, b = host(out1[:used1]), host(out[:used])
        for t1, t in zip(plan.decode_plan(st1), plan.decode_plan(st)):
            assert t.out_offset == t1.out_offset and t.out_len == t1.out_len
            for p1, p in zip(t1.planes, t.planes):
                assert p.codec == p1.codec and p.plane_len == p1.plane_len
                assert b[p.payload_offset: p.payload_offset + p.payload_len] == \
                    b1[p1.payload_offset: p1.payload_offset + p1.payload_len]
        tp = plan.decode_plan(st)
        restored = torch.zeros(tp[-1].out_offset + tp[-1].out_len + 256, dtype=torch.uint8, device="cuda:0")
        assert api.hardware_backend_dispatch_decode_cuda(ids.HARDWARE_BACKEND_LABEL, ids.DECODE_PLAN_LABEL, st,
                                                         out[:used], restored, 0) == total
        r = host(restored)
        for (chain, src), t in zip(items, tp):
            assert r[t.out_offset: t.out_offset + t.out_len] == host(src)
        # the output runs out inside the second batch (the first tensor's
        # payloads fit, the second's do not)
        first = plan.decode_plan(st)[0]
        end0 = max(p.payload_offset + p.payload_len for p in first.planes)
        small = torch.zeros(end0 + 300, dtype=torch.uint8, device="cuda:0")
        with pytest.raises(api.NativeError) as e:
            api.encode_tensors_cuda(items, small, 0, codec=codec)
        assert e.value.rc == -2 and e.value.needed >= used
        big = torch.zeros(e.value.needed, dtype=torch.uint8, device="cuda:0")
        u2, _ = api.encode_tensors_cuda(items, big, 0, codec=codec)
        assert u2 == used
    finally:
        L.ptwm_mi355x_set_encode_batch_bytes(0, 0)


def test_batch_encode_buffer_too_small():
    items = tensors()
    out = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda:0")
    with pytest.raises(api.NativeError) as e:
        api.encode_tensors_cuda(items, out, 0)
    assert e.value.rc == -2
    big = torch.zeros(e.value.needed, dtype=torch.uint8, device="cuda:0")
    used, st = api.encode_tensors_cuda(items, big, 0)
    assert 0 < used <= e.value.needed
