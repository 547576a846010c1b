"""GPU huff_ilv encode, the paths a typical plane does not reach, against
the format's specification encoder (oracle ilv_encode, bytes equal):

- a block whose coded words exceed the encoder's LDS assembly area
  (16 KiB): an all-zero plane with one block of uniform random bytes, so
  that block's symbols carry the longest codes; the other blocks are
  assembled in LDS, that one is written lane by lane;
- stored payloads (tag 0 + shifted copy) and Identity-sized inputs written
  by the batched store kernel, at lengths around the 16-byte vector width
  and into output buffers that are not 16-byte aligned;
- output buffers at any byte alignment (staged).
"""
import sys

import numpy as np
import pytest

import oracle as O
from ptwm_amd import api, ids

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

SEL = ids.PLANE_CODEC_LABEL
OWN = ids.PLANE_CODEC_LABEL


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dev(b: bytes, pad: int = 0):
    a = np.frombuffer(bytes(b), np.uint8)
    t = torch.zeros(len(a) + pad + 1, dtype=torch.uint8, device="cuda:0")
    if len(a):
        t[pad: pad + len(a)].copy_(torch.from_numpy(a.copy()))
    return t[pad: pad + len(a)]


def host(t) -> bytes:
    torch.cuda.synchronize()
    return t.cpu().numpy().tobytes()


def gpu_encode(src: bytes, out_offset: int = 0):
    s = dev(src)
    out = torch.zeros(len(src) + 1 + out_offset, dtype=torch.uint8, device="cuda:0")
    view = out[out_offset:]
    n = api.plane_codec_encode_cuda(SEL, OWN, b"", s, view, 0)
    return host(view)[:n]


def test_block_larger_than_lds_assembly_area():
    n = 16384 * 12
    x = np.zeros(n, np.uint8)
    x[16384 * 5: 16384 * 6] = np.random.default_rng(3).integers(0, 256, 16384)
    x[::97] = 1
    src = x.tobytes()
    want = O.ilv_encode(src)
    assert want[0] == 1  # coded, and the random block alone takes more than 16 KiB
    note(f"encode overflow block n={n} payload={len(want)}")
    assert gpu_encode(src) == want
    dst = torch.zeros(n, dtype=torch.uint8, device="cuda:0")
    got = api.plane_codec_decode_cuda(SEL, OWN, b"", dev(want), dst, 0)
    assert got == n and host(dst) == src


@pytest.mark.parametrize("out_offset", [0, 4, 8])
def test_stored_payloads_at_vector_edges(out_offset):
    rng = np.random.default_rng(17 + out_offset)
    for n in (1, 14, 15, 16, 17, 31, 32, 33, 4095, 16383, 16384, 100_001):
        src = rng.integers(0, 256, n).astype(np.uint8).tobytes()
        want = O.ilv_encode(src)
        assert want[0] == 0, n  # uniform bytes: the stored form
        note(f"encode stored n={n} out_offset={out_offset}")
        assert gpu_encode(src, out_offset) == want, (n, out_offset)


@pytest.mark.parametrize("out_offset", [1, 2, 3])
def test_output_at_any_alignment(out_offset):
    """An output slice that is not 4-byte aligned receives the same payload
    (the encoder writes into aligned staging and copies it)."""
    rng = np.random.default_rng(out_offset)
    for src in (bytes(range(64)), rng.geometric(0.3, 50_000).clip(0, 255).astype(np.uint8).tobytes()):
        note(f"encode into offset {out_offset}, n={len(src)}")
        assert gpu_encode(src, out_offset) == O.ilv_encode(src)
