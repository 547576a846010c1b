"""The allocation-free tensor-level decode
(ptwm_mi355x_dispatch_decode_noalloc_cuda) against the regular one
(ptwm_hardware_backend_v1_dispatch_decode_cuda), through the C ABI.

Two calls in a row, the second with a smaller input, for both GPU-native
codecs, with plane CRC-32 verification: restored bytes equal the regular
entry point's and the inputs, and the library's own allocation counter
(ptwm_mi355x_alloc_calls) does not move across any allocation-free call.
Plans outside the allocation-free route (tensor XXH64, reference-format
planes) are refused with -5, a wrong CRC with -1, as the regular entry point
does; the regular entry point still works after it.  In a fresh process the
call returns -3 before ptwm_mi355x_device_init and decodes after it.
"""
import ctypes as C
import os
import subprocess
import sys

import pytest

from ptwm_amd import api, ids, plan
from ptwm_amd._native import lib

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def plan_id() -> bytes:
    return bytes.fromhex(ids.OWN_IDS[ids.DECODE_PLAN_LABEL])


def noalloc(st: bytes, blob, out) -> int:
    torch.cuda.synchronize()
    pid = plan_id()
    before = lib().ptwm_mi355x_alloc_calls()
    rc = lib().ptwm_mi355x_dispatch_decode_noalloc_cuda(
        1, st, len(st), pid, 32, blob.data_ptr(), blob.numel(), out.data_ptr(), out.numel(), 0)
    assert lib().ptwm_mi355x_alloc_calls() == before, "the allocation-free decode allocated"
    return rc


def regular(st: bytes, blob, out) -> int:
    return api.hardware_backend_dispatch_decode_cuda(ids.HARDWARE_BACKEND_LABEL, ids.DECODE_PLAN_LABEL, st, blob,
                                                     out, 0)


def model(seed: int, scale: int):
    g = torch.Generator(device="cuda:0").manual_seed(seed)
    ts = [
        (plan.CHAIN_IEEE16_SPLIT2, (torch.randn(scale * 16384 + 777, generator=g, device="cuda:0") * 0.02)
         .to(torch.bfloat16)),
        (plan.CHAIN_IEEE16_SPLIT2, (1 + 0.01 * torch.rand(4096, generator=g, device="cuda:0")).to(torch.bfloat16)),
        (plan.CHAIN_IEEE32_SPLIT4, torch.randn(scale * 5000 + 3, generator=g, device="cuda:0") * 0.02),
        (plan.CHAIN_PASSTHROUGH, torch.randint(118, 126, (scale * 20000 + 11,), generator=g, device="cuda:0",
                                               dtype=torch.uint8)),
        (plan.CHAIN_E4M3_NIBBLE, (torch.randn(scale * 30000, generator=g, device="cuda:0") * 40)
         .clamp(-448, 448).to(torch.float8_e4m3fn)),
    ]
    return [(c, t.contiguous().view(torch.uint8)) for c, t in ts]


def encode(items, codec, crc: bool):
    total = sum(t.numel() for _, t in items)
    blob = torch.zeros(2 * total + (1 << 20), dtype=torch.uint8, device="cuda:0")
    used, st = api.encode_tensors_cuda(items, blob, 0, codec=codec)
    plans = plan.decode_plan(st)
    if crc:
        for (chain, raw), t in zip(items, plans):
            if chain in (plan.CHAIN_IEEE16_SPLIT2, plan.CHAIN_IEEE32_SPLIT4, plan.CHAIN_PASSTHROUGH):
                for p, c in zip(t.planes, api.plane_crc32_cuda(chain, raw, 0)):
                    p.crc32 = c
    return blob[:used], plans, total


@pytest.mark.parametrize("codec", ["huff_ilv", "rans_ilv"])
def test_noalloc_matches_regular_two_calls(codec):
    for call, scale in enumerate((40, 3)):   # the second call is smaller
        items = model(100 + call, scale)
        blob, plans, total = encode(items, codec, crc=True)
        st = plan.encode_plan(plans)
        out_len = plans[-1].out_offset + plans[-1].out_len
        a = torch.zeros(out_len, dtype=torch.uint8, device="cuda:0")
        b = torch.full((out_len,), 0xA5, dtype=torch.uint8, device="cuda:0")
        note(f"noalloc {codec} call {call}: {len(items)} tensors, {total} bytes")
        assert regular(st, blob, a) == total
        assert noalloc(st, blob, b) == total
        for (_, raw), t in zip(items, plans):
            sl = slice(t.out_offset, t.out_offset + t.out_len)
            assert torch.equal(b[sl], a[sl]) and torch.equal(b[sl], raw)


def test_noalloc_refuses_what_it_does_not_cover():
    items = model(7, 2)
    blob, plans, total = encode(items, "huff_ilv", crc=True)
    out_len = plans[-1].out_offset + plans[-1].out_len
    out = torch.zeros(out_len, dtype=torch.uint8, device="cuda:0")
    # a wrong plane CRC: InvalidInput, like the regular entry point
    import copy
    bad = copy.deepcopy(plans)
    bad[0].planes[1].crc32 ^= 4
    assert noalloc(plan.encode_plan(bad), blob, out) == -1
    # a tensor XXH64 is outside the allocation-free route: Unsupported
    h = copy.deepcopy(plans)
    h[2].xxh64 = api.xxh64_cuda(items[2][1], 0)
    assert noalloc(plan.encode_plan(h), blob, out) == -5
    # a reference-format plane (exact route): Unsupported
    raw = items[1][1]
    rblob = torch.zeros(2 * raw.numel() + 65536, dtype=torch.uint8, device="cuda:0")
    used, rst = api.encode_tensor_ref_cuda(plan.CHAIN_IEEE16_SPLIT2, [1, 1], 0, raw, rblob, 0)
    rout = torch.zeros(raw.numel(), dtype=torch.uint8, device="cuda:0")
    assert noalloc(rst, rblob[:used], rout) == -5
    # the regular entry point is unaffected by the calls above
    assert regular(plan.encode_plan(plans), blob, out) == total
    for (_, r), t in zip(items, plans):
        assert torch.equal(out[t.out_offset: t.out_offset + t.out_len], r)


FRESH = r"""
import sys
sys.path.insert(0, sys.argv[1])
import numpy as np
import torch
import oracle as O
from ptwm_amd import ids, plan
from ptwm_amd._native import lib

L = lib()
raw = (torch.randn(70001, generator=torch.Generator().manual_seed(5)) * 0.02).to(torch.bfloat16)
raw = raw.view(torch.uint8).numpy().tobytes()
planes = O.chain_forward(O.CHAIN_IEEE16_SPLIT2, raw)
pays = [O.ilv_encode(p) for p in planes]
off1 = (len(pays[0]) + 255) // 256 * 256
blob = pays[0] + bytes(off1 - len(pays[0])) + pays[1]
st = plan.encode_plan([plan.TensorPlan(plan.CHAIN_IEEE16_SPLIT2, 0, len(raw), [
    plan.PlanePlan(ids.CODEC_HUFF_ILV, 0, len(pays[0]), len(planes[0])),
    plan.PlanePlan(ids.CODEC_HUFF_ILV, off1, len(pays[1]), len(planes[1]))])])
d_in = torch.from_numpy(np.frombuffer(blob, np.uint8).copy()).to("cuda:0")
d_out = torch.zeros(len(raw), dtype=torch.uint8, device="cuda:0")
pid = bytes.fromhex(ids.OWN_IDS[ids.DECODE_PLAN_LABEL])
torch.cuda.synchronize()

def call():
    return L.ptwm_mi355x_dispatch_decode_noalloc_cuda(1, st, len(st), pid, 32, d_in.data_ptr(), d_in.numel(),
                                                      d_out.data_ptr(), d_out.numel(), 0)

n0 = L.ptwm_mi355x_alloc_calls()
print("before init", call(), L.ptwm_mi355x_alloc_calls() - n0, flush=True)
print("init", L.ptwm_mi355x_device_init(0), flush=True)
n1 = L.ptwm_mi355x_alloc_calls()
for k in range(2):
    rc = call()
    torch.cuda.synchronize()
    print("call", k, rc, L.ptwm_mi355x_alloc_calls() - n1, d_out.cpu().numpy().tobytes() == raw, flush=True)
"""


def test_noalloc_needs_init_in_a_fresh_process():
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    note("noalloc fresh process: call before and after ptwm_mi355x_device_init")
    r = subprocess.run([sys.executable, "-c", FRESH, root], capture_output=True, text=True, timeout=240)
    note(r.stdout + r.stderr[-2000:])
    assert r.returncode == 0
    lines = [l.split() for l in r.stdout.splitlines()]
    assert lines[0] == ["before", "init", "-3", "0"]   # no context: refused, nothing created
    assert lines[1] == ["init", "0"]
    n = 70001 * 2
    assert lines[2] == ["call", "0", str(n), "0", "True"]
    assert lines[3] == ["call", "1", str(n), "0", "True"]
