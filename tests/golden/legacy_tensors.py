"""Regenerate the input tensors of the reference's legacy fixtures.

Restates the deterministic generator of
``crates/ptwm-core/tests/legacy_fixtures.rs:133-287`` (SplitMix64 with seed
0x5054_574D_4649_5854 for the main tensors, 0x4348_554E_4B45_4421 for the
chunked one; a roughly normal weight from four 24-bit uniforms in f32
arithmetic; bf16 by truncation, f16 by the fixture's own truncating
conversion).  ``legacy_xxh64.json`` holds the reference's EXPECTED table
(``legacy_fixtures.rs:63-123``: tensor name, decoded length, xxh64 seed 0),
which pins the XXH64 implementations here and on the GPU.
"""
from __future__ import annotations

import json
import os

import numpy as np

MASK = (1 << 64) - 1
F = np.float32


class SplitMix64:
    def __init__(self, seed: int):
        self.s = seed & MASK

    def next_u64(self) -> int:
        self.s = (self.s + 0x9E3779B97F4A7C15) & MASK
        z = self.s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK
        return z ^ (z >> 31)

    def weight(self) -> np.float32:
        s = F(0.0)
        for _ in range(4):
            s = F(s + F(self.next_u64() >> 40) / F(1 << 24))
        return F((s - F(2.0)) * F(0.05))


def _bits(v: np.float32) -> int:
    return int(np.array([v], np.float32).view(np.uint32)[0])


def _bf16(v) -> bytes:
    return (_bits(v) >> 16).to_bytes(2, "little")


def _f16(v) -> bytes:
    b = _bits(v)
    sign = (b >> 16) & 0x8000
    exp = ((b >> 23) & 0xFF) - 127 + 15
    if exp <= 0:
        return sign.to_bytes(2, "little")
    return (sign | (exp << 10) | ((b >> 13) & 0x3FF)).to_bytes(2, "little")


def _bf16_tensor(rng, n):
    return b"".join(_bf16(rng.weight()) for _ in range(n))


def tensors() -> dict[str, bytes]:
    """name -> raw bytes, in the generator's order (legacy_fixtures.rs:191-287)."""
    rng = SplitMix64(0x5054574D46495854)
    out = {"model.layers.0.q.weight": _bf16_tensor(rng, 8 * 32)}
    out["model.layers.0.k.weight"] = b"".join(_f16(rng.weight()) for _ in range(8 * 32))
    out["model.norm.weight"] = b"".join(
        np.array([F(F(1.0) + rng.weight())], np.float32).tobytes() for _ in range(4 * 32))
    fp8 = bytearray()
    for _ in range(256):
        r = rng.next_u64()
        exp = 3 + r % 5
        fp8.append(((r >> 8) & 0x80) | (exp << 3) | ((r >> 16) & 0x07))
    out["model.layers.0.mlp.fp8.weight"] = bytes(fp8)
    out["model.embed.int8"] = bytes(((rng.next_u64() % 9) - 4) & 0xFF for _ in range(256))
    for name in ("model.layers.0.q.scale", "model.layers.0.k.scale"):
        b = bytearray()
        for _ in range(64):
            prev = 0x80
            for _ in range(32):
                prev = (prev + rng.next_u64() % 3 - 1) & 0xFF
                b.append(prev)
        out[name] = bytes(b)
    res = bytearray(_bf16_tensor(rng, 4 * 32))
    for i in range(0, len(res), 3):
        res[i] = 0
    out["model.layers.1.q.weight"] = bytes(res)
    rng2 = SplitMix64(0x4348554E4B454421)
    out["model.layers.2.chunked.weight"] = _bf16_tensor(rng2, 16 * 32)
    return out


def expected() -> dict[str, tuple[int, int]]:
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "legacy_xxh64.json")) as f:
        return {k: (v[0], int(v[1], 16)) for k, v in json.load(f).items()}
