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


def test_batch_encode_buffer_too_small():
    items = tensors()
    out = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda:0")
    with pytest.raises(api.NativeError) as e:
        api.encode_tensors_cuda(items, out, 0)
    assert e.value.rc == -2
    big = torch.zeros(e.value.needed, dtype=torch.uint8, device="cuda:0")
    used, st = api.encode_tensors_cuda(items, big, 0)
    assert 0 < used <= e.value.needed
