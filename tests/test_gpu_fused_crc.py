"""Plane CRC-32 computed inside the fused huff_ilv decode (whole 16 KiB
blocks of each plane folded while the planes are merged, the partial last
block from the restored tensor, then combined), checked the way the
reference checks a decoded plane (container.rs:2154-2159: crc32fast of the
plane bytes, a mismatch is InvalidContainer):

- one plan mixing chains (bf16 split2, fp32 split4, passthrough), plane
  lengths that are exact multiples of the block, under one block, one
  element, and ragged; tensors with and without CRCs; rans_ilv tensors
  (standalone CRC kernel) in the same plan;
- every plane's expected CRC is the oracle's CRC-32 of the oracle's plane
  bytes, so a dropped block, a wrong advance or a wrong byte rotation of
  the exponent plane fails the decode;
- flipping one bit of any single plane's CRC makes the decode fail.
"""
import sys

import numpy as np
import pytest

import oracle as O
from ptwm_amd import api, ids, plan

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def host(t) -> bytes:
    torch.cuda.synchronize()
    return t.cpu().numpy().tobytes()


def _items(seed):
    g = torch.Generator(device="cuda:0").manual_seed(seed)
    bf = lambda n: (torch.randn(n, generator=g, device="cuda:0") * 0.02).to(torch.bfloat16)  # noqa: E731
    f32 = lambda n: torch.randn(n, generator=g, device="cuda:0") * 3.0  # noqa: E731
    u8 = lambda n: torch.randint(100, 140, (n,), generator=g, device="cuda:0", dtype=torch.uint8)  # noqa: E731
    out = [
        (plan.CHAIN_IEEE16_SPLIT2, bf(3 * 16384)),       # whole blocks only
        (plan.CHAIN_IEEE16_SPLIT2, bf(5 * 16384 + 77)),  # ragged last block
        (plan.CHAIN_IEEE16_SPLIT2, bf(1)),
        (plan.CHAIN_IEEE16_SPLIT2, bf(16383)),
        (plan.CHAIN_IEEE32_SPLIT4, f32(2 * 16384 + 4000)),
        (plan.CHAIN_IEEE32_SPLIT4, f32(16384)),
        (plan.CHAIN_PASSTHROUGH, u8(200_001)),
        (plan.CHAIN_IEEE16_SPLIT2, bf(40_000)),          # no CRC on this one
    ]
    return [(c, t.contiguous().view(torch.uint8)) for c, t in out]


def _encode(items, codec):
    total = sum(t.numel() for _, t in items)
    out = torch.zeros(total * 2 + (1 << 20), dtype=torch.uint8, device="cuda:0")
    used, st = api.encode_tensors_cuda(items, out, 0, codec=codec)
    return host(out[:used]), plan.decode_plan(st)


def _plan_with_crcs(seed):
    huff = _items(seed)
    rans = _items(seed + 1)[:3]
    hb, ht = _encode(huff, "huff_ilv")
    rb, rt = _encode(rans, "rans_ilv")
    # one input buffer and one output buffer for both groups
    boff = (len(hb) + 255) // 256 * 256
    ooff = (ht[-1].out_offset + ht[-1].out_len + 255) // 256 * 256
    for t in rt:
        t.out_offset += ooff
        for p in t.planes:
            p.payload_offset += boff
    blob = hb + b"\0" * (boff - len(hb)) + rb
    tensors = ht + rt
    datas = [host(s) for _, s in huff + rans]
    for i, (t, d) in enumerate(zip(tensors, datas)):
        if i == len(huff) - 1:
            continue  # a tensor without CRCs in the middle of the plan
        for p, pb in zip(t.planes, O.chain_forward(t.chain, d)):
            p.crc32 = O.crc32(pb)
    return blob, tensors, datas


def _decode(st, blob_dev, out):
    return api.hardware_backend_dispatch_decode_cuda(ids.HARDWARE_BACKEND_LABEL, ids.DECODE_PLAN_LABEL, st,
                                                     blob_dev, out, 0)


def test_fused_crc_plan_verifies_and_detects_each_plane():
    blob, tensors, datas = _plan_with_crcs(31)
    note(f"fused crc: {len(tensors)} tensors, blob {len(blob)} bytes")
    blob_dev = torch.from_numpy(np.frombuffer(blob, np.uint8).copy()).to("cuda:0")
    total = tensors[-1].out_offset + tensors[-1].out_len
    out = torch.zeros(total, dtype=torch.uint8, device="cuda:0")
    n = _decode(plan.encode_plan(tensors), blob_dev, out)
    got = host(out)
    written = sum(t.out_len for t in tensors)
    assert n == written
    for t, d in zip(tensors, datas):
        assert got[t.out_offset: t.out_offset + t.out_len] == d
    # one wrong plane CRC at a time: InvalidInput (rc -1)
    for ti, t in enumerate(tensors):
        for pi, p in enumerate(t.planes):
            if p.crc32 is None:
                continue
            note(f"fused crc: flip tensor {ti} plane {pi}")
            p.crc32 ^= 1 << (pi + ti) % 32
            with pytest.raises(Exception) as ei:
                _decode(plan.encode_plan(tensors), blob_dev, out)
            assert getattr(ei.value, "rc", None) == -1, (ti, pi)
            p.crc32 ^= 1 << (pi + ti) % 32
    # and the restored plan still verifies afterwards (partials rewritten)
    assert _decode(plan.encode_plan(tensors), blob_dev, out) == written


def test_fused_crc_llama_like_tensor_repeated():
    """A 16 Mi-element bf16 tensor (1024 blocks per plane), decoded twice in
    a row with CRCs: the second call's partials overwrite the first's."""
    g = torch.Generator(device="cuda:0").manual_seed(5)
    x = (torch.randn(1 << 24, generator=g, device="cuda:0") * 0.02).to(torch.bfloat16).view(torch.uint8)
    blob, tp = _encode([(plan.CHAIN_IEEE16_SPLIT2, x)], "huff_ilv")
    d = host(x)
    for p, pb in zip(tp[0].planes, O.chain_forward(plan.CHAIN_IEEE16_SPLIT2, d)):
        p.crc32 = O.crc32(pb)
    blob_dev = torch.from_numpy(np.frombuffer(blob, np.uint8).copy()).to("cuda:0")
    out = torch.zeros(len(d), dtype=torch.uint8, device="cuda:0")
    for k in range(2):
        note(f"fused crc 32 MiB bf16 call {k}")
        out.zero_()
        assert _decode(plan.encode_plan(tp), blob_dev, out) == len(d)
        assert host(out) == d
