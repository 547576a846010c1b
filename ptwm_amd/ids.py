"""Canonical ids (32-byte blake3) this library recognises.

Built-in ids are ``blake3([0xBB]*32 || 0 || name || 0 || version)``
(crates/ptwm-core/src/extension/id.rs:21-30, extension/mod.rs:36,
extension/builtins.rs:18-27); the values below are those derivations, and
tests recompute them.  This extension's own ids use the all-zero author key
of the reference's in-tree bundles (extensions/*/manifest.toml).
"""

from __future__ import annotations

import functools

BUILTIN_IDS = {
    ("identity", "1.1.0"): "fc2dea1265e3394c57c2df3b868b732ccaa1ee876bd4b1ce27d38f842c6112b5",
    ("huffman", "1.1.0"): "614155b5a8c9efb689219bcca3cbf7855e29d3023208ce61cca7a36849248e33",
    ("rans", "1.1.0"): "39c875ef9793a9c5ebe199116debac4c9d5388b8b7cf2fe6b575845f0ca1624e",
    ("identity", "1.0.0"): "eb31edfe6fd156b309010ca750571766fc8ae6e4056bc2b4a228679922edea30",
    ("huffman", "1.0.0"): "571e8fae548f0db5faa961fb65ba5ea2443bdb1e95dac04fbf1d5d97228ec945",
    ("rans", "1.0.0"): "87c8ca053fbd0646c07d18da4d0396a92550eb6d44bcd4e461538902874d4bc7",
}
CURRENT_BUILTIN_VERSION = "1.1.0"   # extension/builtins.rs:19 (crate version)

PLANE_CODEC_LABEL = "io.ptwm.mi355x.plane_codec"            # huff_ilv
RANS_CODEC_LABEL = "io.ptwm.mi355x.plane_codec.rans"        # rans_ilv
HARDWARE_BACKEND_LABEL = "io.ptwm.mi355x.hardware_backend"
DECODE_PLAN_LABEL = "io.ptwm.mi355x.decode_plan"
OWN_VERSION = "0.1.0"
OWN_IDS = {
    PLANE_CODEC_LABEL: "cfd8cc03483eb4a43cdddb4b3cbf95b32e0a3f0e17e5ec85a0b52de04e8caf04",
    HARDWARE_BACKEND_LABEL: "a432dc02f57030b41a3660762bbcec5668cde8abbc807999d56ca0a3304d39cf",
    DECODE_PLAN_LABEL: "1b0e48b156b01d0d733a5aa62a90bcbde34945ff024d8d8e56cb714a48c6e770",
    RANS_CODEC_LABEL: "968f8be9f06b14b33fcd066622493f1101954d074c25d63e78380d33708fe1f5",
}

# codec wire ids (crates/ptwm-core/src/codec.rs:3-23)
CODEC_IDENTITY = 0x0000
CODEC_HUFFMAN = 0x0001
CODEC_RANS = 0x0003
CODEC_ZSTD = 0x0004
CODEC_HUFF_ILV = 0x7F01            # this library's GPU-native codecs
CODEC_RANS_ILV = 0x7F02
CODEC_NAMES = {"identity": CODEC_IDENTITY, "huffman": CODEC_HUFFMAN, "rans": CODEC_RANS}


@functools.lru_cache(maxsize=256)
def resolve_codec_selector(selector: str) -> bytes:
    """Mirror of extension/resolve.rs:34-75 over the ids known here: a
    ``blake3:<hex>`` or bare 64-hex id, a built-in codec name, or one of
    this extension's labels.  (Results are cached: selectors are a handful
    of constants, resolved on every device call.)"""
    s = selector.strip()
    hexpart = s[7:] if s.startswith("blake3:") else s
    if len(hexpart) == 64:
        try:
            return bytes.fromhex(hexpart)
        except ValueError:
            pass
    if s in CODEC_NAMES:
        return bytes.fromhex(BUILTIN_IDS[(s, CURRENT_BUILTIN_VERSION)])
    if s in OWN_IDS:
        return bytes.fromhex(OWN_IDS[s])
    raise LookupError(f"no codec or contribution matches selector {selector!r}")


def codec_wire_id(canonical: bytes) -> int:
    h = canonical.hex()
    for (name, _v), hx in BUILTIN_IDS.items():
        if hx == h:
            return CODEC_NAMES[name]
    if h == OWN_IDS[PLANE_CODEC_LABEL]:
        return CODEC_HUFF_ILV
    if h == OWN_IDS[RANS_CODEC_LABEL]:
        return CODEC_RANS_ILV
    raise LookupError(f"unknown codec id {h}")
