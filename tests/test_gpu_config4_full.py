"""Config 4 at full size: the Llama-3-8B-shaped bf16 model (290 tensors,
16 060 514 304 bytes) encoded by the GPU batch encoder into one plan that
carries every plane's CRC-32 and every tensor's XXH64, then restored by ONE
tensor-level decode call with both verified, as the reference's container
decode verifies them (container.rs:2154-2159 plane CRC, :2185-2194 payload
hash; emitted by default, python/ptwm/_config.py:177-179).

- every restored tensor equals its input (torch.equal on the device);
- one tensor of every shape class (the 1 GiB embedding, attention q/o and
  k/v, MLP gate/up and down, the norms) is checked against the CPU oracle:
  each plane payload decoded by the format specification (por_ilv_decode)
  and merged by the reference's fused inverse (fusion.rs), plane CRC-32 by
  the oracle's crc32fast restatement, tensor XXH64 by the oracle's xxhash
  restatement;
- a plan with one wrong CRC, or one wrong hash, is rejected (-1);
- the model as a file ("multi-tensor .ptwm container"):
  the GPU-encoded payloads written by the library's container writer as a
  compact container (\\x89PTWC, 290 records with shapes, plane CRC-32s and
  XXH64s), re-opened by ptwm_mi355x_container_plan, restored in one call on
  the GPU and the shape-class sample decoded from the file by the oracle;
  the same model encoded on the GPU in the reference's own format (Huffman
  planes in 256 KiB chunk frames, python/ptwm/_config.py:151), whose
  payloads equal the oracle's restatement of the reference encoder on the
  sample, written, re-opened and restored the same way.
"""
import sys

import numpy as np
import pytest

import bench
import oracle as O
from ptwm_amd import api, ids, plan

import file_writer
import plan_oracle

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


# one tensor of every shape class of the model
SAMPLE = ["model.embed_tokens.weight", "model.layers.0.self_attn.q_proj.weight",
          "model.layers.7.self_attn.k_proj.weight", "model.layers.13.input_layernorm.weight",
          "model.layers.31.post_attention_layernorm.weight", "model.layers.20.mlp.down_proj.weight",
          "model.layers.26.mlp.up_proj.weight", "model.layers.5.self_attn.o_proj.weight"]
DT_BF16 = 6  # dtype.rs:79-103


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


def test_sample_covers_every_shape_class():
    classes = {(tuple(sh), k) for _, sh, k in bench.llama8b_shapes()}
    by_name = {n: (tuple(sh), k) for n, sh, k in bench.llama8b_shapes()}
    assert {by_name[n] for n in SAMPLE} == classes


def host_np(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def to_device(a):
    t = torch.empty(max(1, a.size), dtype=torch.uint8, device="cuda:0")
    t[: a.size].copy_(torch.from_numpy(a))
    return t[: a.size]


def write_and_restore(names, items, entries, payloads, label):
    """Write the model, re-open the file, restore it on the GPU in one call
    with every CRC and hash checked; returns the file and its plan."""
    data = api.container_write(file_writer.write_tensors(entries), payloads=payloads, as_array=True)
    note(f"config 4 {label}: compact container written, {data.size} bytes")
    assert data[:9].tobytes() == b"\x89PTWC\r\n\x1a\n"
    plan_bytes, ents, out_len = api.container_plan(data)
    assert [e.name for e in ents] == names
    assert all(e.status == 0 and e.plan_index >= 0 and e.crc_checked and e.hash_checked for e in ents)
    assert out_len >= R_TOTAL
    src = to_device(data)
    restored = torch.zeros(out_len, dtype=torch.uint8, device="cuda:0")
    assert dispatch(plan_bytes, src, restored) == R_TOTAL
    for e, (_, raw) in zip(ents, items):
        assert torch.equal(restored[e.out_offset:e.out_offset + e.orig_size], raw), e.name
    note(f"config 4 {label}: file re-opened, 290 tensors restored bit-exact, CRC-32 + XXH64 verified")
    del src, restored
    return data, plan_bytes, ents


def oracle_sample_from_file(names, items, data, plan_bytes, ents, label):
    tp = plan.decode_plan(plan_bytes)
    for name in SAMPLE:
        e = ents[names.index(name)]
        got = plan_oracle.decode_tensor(data, tp[e.plan_index])  # checks the CRCs and the XXH64 too
        assert got == host(items[names.index(name)][1]), name
    note(f"config 4 {label}: shape-class sample decoded from the file by the oracle")


def test_config4_as_a_file(model):
    names, items, blob, plans = model
    shapes = {n: list(sh) for n, sh, _ in bench.llama8b_shapes()}
    payloads = host_np(blob)
    entries = [(n, DT_BF16, shapes[n], t) for n, t in zip(names, plans)]
    data, plan_bytes, ents = write_and_restore(names, items, entries, payloads, "huff_ilv")
    del payloads
    oracle_sample_from_file(names, items, data, plan_bytes, ents, "huff_ilv")


def test_config4_reference_format_file(model):
    names, items, _, plans = model
    shapes = {n: list(sh) for n, sh, _ in bench.llama8b_shapes()}
    codecs, chunk = bench.REF_FORMATS["c4"]["w"]
    cap = R_TOTAL + 65536 * len(items) + (1 << 20)
    blob = torch.empty(cap, dtype=torch.uint8, device="cuda:0")
    off, entries = 0, []
    for name, (chain, raw), p0 in zip(names, items, plans):
        used, st = api.encode_tensor_ref_cuda(chain, codecs, chunk, raw, blob[off:], 0)
        t = plan.decode_plan(st)[0]
        for p, q in zip(t.planes, p0.planes):
            p.payload_offset += off
            p.crc32 = q.crc32  # the same planes as the huff_ilv encode's: CRC-32s by plane_crc32_cuda
        t.xxh64 = p0.xxh64
        entries.append((name, DT_BF16, shapes[name], t))
        off = (off + used + 255) // 256 * 256
    note(f"config 4 reference format: {off} bytes encoded on the GPU")
    payloads = host_np(blob[:off])
    del blob
    # the GPU encoder's payloads are the reference encoder's (oracle restatement)
    for name in SAMPLE:
        i = names.index(name)
        t = entries[i][3]
        for p, pl in zip(t.planes, O.chain_forward(plan.CHAIN_IEEE16_SPLIT2, host(items[i][1]))):
            pay, ent = O.encode_plane_chunked(codecs[0], pl, chunk)
            assert p.codec == codecs[0] and p.crc32 == O.crc32(pl), name
            assert payloads[p.payload_offset:p.payload_offset + p.payload_len].tobytes() == pay, name
            assert [tuple(c) for c in p.chunks] == [tuple(int(v) for v in e) for e in ent], name
    note("config 4 reference format: shape-class sample payloads == oracle encode")
    data, plan_bytes, ents = write_and_restore(names, items, entries, payloads, "reference format")
    del payloads
    oracle_sample_from_file(names, items, data, plan_bytes, ents, "reference format")
