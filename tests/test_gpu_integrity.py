"""GPU integrity checks against the CPU oracle: plane CRC-32 and tensor XXH64.

The reference verifies each decoded plane with crc32fast (CRC-32/ISO-HDLC,
container.rs:2154-2159) and each restored tensor with xxh64 seed 0
(container.rs:2185-2194, compact.rs:441-445).  The oracle's por_crc32 /
por_xxh64 are pinned against zlib.crc32 and the reference's golden
EXPECTED xxh64 tables on the CPU side; here the GPU kernels must equal them,
and a decode plan carrying CRCs / hashes must accept the right values and
reject a wrong one with InvalidInput (-1), as the reference's
InvalidContainer("plane CRC mismatch" / "tensor payload hash mismatch").
"""
import sys

import numpy as np
import pytest

import oracle as O
from ptwm_amd import api, ids, plan

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

LENGTHS = [0, 1, 3, 4, 7, 8, 15, 16, 17, 31, 32, 33, 63, 64, 255, 256, 4095, 4096, 4097, 65535, 65536, 65537,
           1 << 20, (1 << 20) + 5, 3 * (1 << 20) + 4093, 20 * (1 << 20) + 7]


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dev_bytes(b: bytes):
    t = torch.empty(max(1, len(b)), dtype=torch.uint8, device="cuda:0")
    if b:
        t[: len(b)].copy_(torch.from_numpy(np.frombuffer(b, np.uint8).copy()))
    return t[: len(b)]


def rnd(n, seed):
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8).tobytes()


@pytest.mark.parametrize("n", LENGTHS)
def test_crc32_plane_matches_oracle(n):
    note(f"crc32 passthrough n={n}")
    data = rnd(n, n)
    got = api.plane_crc32_cuda(plan.CHAIN_PASSTHROUGH, dev_bytes(data), 0)
    assert got == [O.crc32(data)]


@pytest.mark.parametrize("chain,elems", [(plan.CHAIN_IEEE16_SPLIT2, e) for e in (0, 1, 15, 16, 4096, 70001, 1 << 21)]
                         + [(plan.CHAIN_IEEE32_SPLIT4, e) for e in (1, 17, 4097, 300003)])
def test_crc32_of_planes_from_restored_tensor(chain, elems):
    note(f"crc32 chain={chain} elems={elems}")
    data = rnd(elems * plan.CHAIN_RATIO[chain], 7 + elems)
    got = api.plane_crc32_cuda(chain, dev_bytes(data), 0)
    assert got == [O.crc32(p) for p in O.chain_forward(chain, data)]


@pytest.mark.parametrize("n", LENGTHS + [64 * 32 - 1, 64 * 32, 64 * 32 + 1, 64 * 32 * 5 + 40])
def test_xxh64_matches_oracle(n):
    note(f"xxh64 n={n}")
    data = rnd(n, 100 + n)
    assert api.xxh64_cuda(dev_bytes(data), 0) == O.xxh64(data)


def test_xxh64_reference_golden_table():
    """The reference's EXPECTED (length, xxh64) of its legacy fixture tensors."""
    import os
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
    import legacy_tensors as G
    t = G.tensors()
    for name, (n, h) in G.expected().items():
        note(f"xxh64 golden {name}")
        assert api.xxh64_cuda(dev_bytes(t[name]), 0) == h, name


def _bf16(shape, seed):
    return (torch.randn(*shape, generator=torch.Generator().manual_seed(seed)) * 0.02).to(torch.bfloat16)


def _encode(kind, data_dev, chain):
    out = torch.zeros(2 * data_dev.numel() + (1 << 20), dtype=torch.uint8, device="cuda:0")
    if kind == "ilv":
        used, st = api.encode_tensor_cuda(chain, data_dev, out, 0)
    else:
        codecs = [O.CODEC_HUFFMAN] * plan.CHAIN_PLANES[chain]
        used, st = api.encode_tensor_ref_cuda(chain, codecs, kind == "ref-chunked" and 65536 or 0, data_dev, out, 0)
    return out[:used], plan.decode_plan(st)[0]


CASES = [("ilv", plan.CHAIN_IEEE16_SPLIT2), ("ref", plan.CHAIN_IEEE16_SPLIT2), ("ref-chunked", plan.CHAIN_IEEE32_SPLIT4),
         ("ilv", plan.CHAIN_E4M3_NIBBLE), ("ref", plan.CHAIN_NIBBLE_SPLIT), ("ilv", plan.CHAIN_PASSTHROUGH)]


@pytest.mark.parametrize("kind,chain", CASES, ids=[f"{k}-c{c}" for k, c in CASES])
def test_plan_with_crc_and_hash_verifies(kind, chain):
    note(f"plan crc+hash {kind} chain={chain}")
    if chain in (plan.CHAIN_IEEE16_SPLIT2,):
        data = _bf16((512, 1000), 3).view(torch.uint8).reshape(-1).numpy().tobytes()
    elif chain == plan.CHAIN_IEEE32_SPLIT4:
        data = (torch.randn(300, 700, generator=torch.Generator().manual_seed(4)) * 0.02).view(torch.uint8)
        data = data.reshape(-1).numpy().tobytes()
    else:
        x = np.random.default_rng(5).geometric(0.3, 400_000).clip(0, 255).astype(np.uint8)
        data = x.tobytes()
    src = dev_bytes(data)
    blob, t = _encode(kind, src, chain)
    planes = O.chain_forward(chain, data)
    for p, pp in zip(planes, t.planes):
        pp.crc32 = O.crc32(p)
    t.xxh64 = O.xxh64(data)
    out = torch.zeros(len(data), dtype=torch.uint8, device="cuda:0")
    st = plan.encode_plan([t])
    n = api.hardware_backend_dispatch_decode_cuda(ids.HARDWARE_BACKEND_LABEL, ids.DECODE_PLAN_LABEL, st, blob, out, 0)
    torch.cuda.synchronize()
    assert n == len(data) and out.cpu().numpy().tobytes() == data
    # a wrong plane CRC or a wrong tensor hash is InvalidInput
    for which in ["crc", "hash"]:
        t2 = plan.decode_plan(st)[0]
        if which == "crc":
            t2.planes[-1].crc32 ^= 1
        else:
            t2.xxh64 ^= 1 << 40
        with pytest.raises(Exception) as ei:
            api.hardware_backend_dispatch_decode_cuda(ids.HARDWARE_BACKEND_LABEL, ids.DECODE_PLAN_LABEL,
                                                      plan.encode_plan([t2]), blob, out, 0)
        assert getattr(ei.value, "rc", None) == -1, which
