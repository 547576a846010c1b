"""Config 4 at full size: the Llama-3-8B-shaped bf16 model (290 tensors,
16 060 514 304 bytes) encoded by the GPU batch encoder into one plan that
carries every plane's CRC-32 and every tensor's XXH64, then restored by ONE
tensor-level decode call with both verified, as the reference's container
decode verifies them (container.rs:2154-2159 plane CRC, :2185-2194 payload
hash; emitted by default, python/ptwm/_config.py:177-179).

- every restored tensor equals its input (torch.equal on the device);
- a sample of tensors is checked against the CPU oracle: each plane payload
  decoded by the format specification (por_ilv_decode) and merged by the
  reference's fused inverse (fusion.rs), plane CRC-32 by the oracle's
  crc32fast restatement, tensor XXH64 by the oracle's xxhash restatement;
- a plan with one wrong CRC, or one wrong hash, is rejected (-1).
"""
import sys

import numpy as np
import pytest

import bench
import oracle as O
from ptwm_amd import api, ids, plan

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

R_TOTAL = 16_060_514_304


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def host(t) -> bytes:
    torch.cuda.synchronize()
    return t.cpu().numpy().tobytes()


@pytest.fixture(scope="module")
def model():
    shapes = bench.llama8b_shapes()
    assert len(shapes) == 290
    items = [(plan.CHAIN_IEEE16_SPLIT2, bench.gen_tensor(kind, shape, 1000 + i))
             for i, (_, shape, kind) in enumerate(shapes)]
    total = sum(t.numel() for _, t in items)
    assert total == R_TOTAL
    note(f"config 4: {len(items)} tensors, {total} bytes generated")
    blob = torch.empty(total + 65536 * len(items) + (1 << 20), dtype=torch.uint8, device="cuda:0")
    used, st = api.encode_tensors_cuda(items, blob, 0)
    plans = plan.decode_plan(st)
    note(f"config 4: encoded to {used} bytes (ratio {used / total:.4f})")
    for (chain, raw), t in zip(items, plans):
        for p, c in zip(t.planes, api.plane_crc32_cuda(chain, raw, 0)):
            p.crc32 = c
        t.xxh64 = api.xxh64_cuda(raw, 0)
    note("config 4: plane CRC-32 and tensor XXH64 computed")
    yield [n for n, _, _ in shapes], items, blob[:used], plans
    del blob, items


def dispatch(st, blob, out):
    return api.hardware_backend_dispatch_decode_cuda(ids.HARDWARE_BACKEND_LABEL, ids.DECODE_PLAN_LABEL, st, blob,
                                                     out, 0)


def test_config4_full_model_one_call_crc_and_hash_verified(model):
    names, items, blob, plans = model
    out_len = plans[-1].out_offset + plans[-1].out_len
    restored = torch.zeros(out_len, dtype=torch.uint8, device="cuda:0")
    n = dispatch(plan.encode_plan(plans), blob, restored)
    assert n == R_TOTAL
    for name, (_, raw), t in zip(names, items, plans):
        assert torch.equal(restored[t.out_offset: t.out_offset + t.out_len], raw), name
    note("config 4: 290 tensors restored bit-exact with CRC-32 + XXH64 verified")


SAMPLE = ["model.layers.0.self_attn.q_proj.weight", "model.layers.7.self_attn.k_proj.weight",
          "model.layers.13.input_layernorm.weight", "model.layers.31.post_attention_layernorm.weight",
          "model.layers.20.mlp.down_proj.weight"]


def test_config4_sampled_tensors_match_oracle(model):
    names, items, blob, plans = model
    for name in SAMPLE:
        i = names.index(name)
        raw, t = items[i][1], plans[i]
        data = host(raw)
        planes = []
        for p in t.planes:
            payload = host(blob[p.payload_offset: p.payload_offset + p.payload_len])
            if p.codec == 0x7F01:
                planes.append(O.ilv_decode(payload, p.plane_len))
            else:
                assert p.codec == 0 and len(payload) == p.plane_len
                planes.append(payload)
        for p, pl in zip(t.planes, planes):
            assert O.crc32(pl) == p.crc32, name
        assert O.chain_inverse(plan.CHAIN_IEEE16_SPLIT2, planes) == data, name
        assert O.xxh64(data) == t.xxh64, name
        note(f"config 4 oracle check {name}: {len(data)} bytes, planes {[hex(p.codec) for p in t.planes]}")


@pytest.mark.parametrize("what", ["crc", "hash"])
def test_config4_wrong_integrity_value_rejected(model, what):
    import copy

    names, items, blob, plans = model
    bad = copy.deepcopy(plans)
    i = names.index("model.layers.17.mlp.up_proj.weight")
    if what == "crc":
        bad[i].planes[1].crc32 ^= 1
    else:
        bad[i].xxh64 ^= 1 << 40
    out_len = bad[-1].out_offset + bad[-1].out_len
    restored = torch.zeros(out_len, dtype=torch.uint8, device="cuda:0")
    with pytest.raises(api.NativeError) as e:
        dispatch(plan.encode_plan(bad), blob, restored)
    assert e.value.rc == -1
