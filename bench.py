"""Decode-throughput benchmark of the MI355X plane-codec path.

``python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload llama8b+crc|llama8b|fp8|...]``

A "step" restores every tensor of the workload from its compressed planes,
resident in HBM, through the library's tensor-level entry point
(``ptwm_hardware_backend_v1_dispatch_decode_cuda``): entropy decode plus the
inverse chain (merge + bit revert) in one fused kernel per chain and, for the
default headline (config 4, ``llama8b+crc``), the CRC-32 of every decoded
plane checked against the plan inside the timed region, as the reference's
container decode does by default (container.rs:2154-2159,
_config.py:179).  Inputs are synthetic tensors of the BASELINE.json shapes,
generated on the GPU from fixed seeds and encoded by the library's own GPU
encoder (huff_ilv planes, Identity when coding does not shrink a plane).
Every step's output is checked bit-exact against the original tensors after
the timed region.

Prints one JSON line: ``value`` = restored GB/s (whole job, one GPU),
``roofline`` for the dominant kernel (HIP events on the library stream),
``config.hash_verified`` = the same decode with every tensor's XXH64 also
verified, ``config.secondary`` = the same bytes without verification, the
other configs and the reference-format routes, and ``cpu_baseline`` = the C
restatement of the reference CPU decoder (4-segment Huffman decode + fused
inverse, tensors over threads) on a bounded sample of the same workload,
timed on this host.
"""
from __future__ import annotations

import argparse
import ctypes as C
import gc
import json
import re
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0

# Measured HBM bytes per launch of the workload's dominant kernel: the
# copy-calibrated FETCH_SIZE + WRITE_SIZE of two rocprofv3 --pmc runs of this
# script, recorded (with the commands and raw counters) in these summaries.
TRAFFIC_PROFILES = {"llama8b": "profiles/ilv_decode_kernel_bf16_llama8b.md",
                    "llama8b+crc": "profiles/ilv_decode_kernel_crc_llama8b_crc.md"}


def measured_traffic(workload: str):
    rel = TRAFFIC_PROFILES.get(workload)
    if not rel or not os.path.exists(os.path.join(ROOT, rel)):
        return None, None
    with open(os.path.join(ROOT, rel)) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1]), rel
    return None, None


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def llama8b_shapes():
    """Llama-3-8B-shaped bf16 model (290 tensors)."""
    shapes = [("model.embed_tokens.weight", (128256, 4096), "w")]
    for i in range(32):
        p = f"model.layers.{i}."
        shapes += [
            (p + "self_attn.q_proj.weight", (4096, 4096), "w"),
            (p + "self_attn.k_proj.weight", (1024, 4096), "w"),
            (p + "self_attn.v_proj.weight", (1024, 4096), "w"),
            (p + "self_attn.o_proj.weight", (4096, 4096), "w"),
            (p + "mlp.gate_proj.weight", (14336, 4096), "w"),
            (p + "mlp.up_proj.weight", (14336, 4096), "w"),
            (p + "mlp.down_proj.weight", (4096, 14336), "w"),
            (p + "input_layernorm.weight", (4096,), "n"),
            (p + "post_attention_layernorm.weight", (4096,), "n"),
        ]
    shapes.append(("lm_head.weight", (128256, 4096), "w"))
    return shapes


class Workload:
    def __init__(self, name):
        self.name = name
        self.tensors = []        # (raw uint8 device tensor, chain, reference codecs or None)
        self.blob = None
        self.plan_bytes = b""
        self.out_len = 0
        self.comp_bytes = 0
        self.restored = 0
        self.kernel = ""


def gen_tensor(kind, shape, seed):
    import torch

    g = torch.Generator(device="cuda:0").manual_seed(seed)
    if kind == "w":            # N(0, 0.02) bf16
        return (torch.randn(shape, generator=g, device="cuda:0") * 0.02).to(torch.bfloat16).view(torch.uint8).reshape(-1)
    if kind == "n":            # RMSNorm weights ~ 1.0 +/- 0.01
        return (1 + 0.01 * (2 * torch.rand(shape, generator=g, device="cuda:0") - 1)).to(torch.bfloat16).view(
            torch.uint8).reshape(-1)
    if kind == "fp8":          # per-row absmax scaled N(0,1) cast to e4m3 (config 3)
        x = torch.randn(shape, generator=g, device="cuda:0")
        x = x / x.abs().amax(1, keepdim=True) * 448
        return x.to(torch.float8_e4m3fn).view(torch.uint8).reshape(-1)
    if kind == "fp32o":        # N(0,0.02) fp32 with 1% x50 outliers (config 2)
        w = torch.randn(shape, generator=g, device="cuda:0") * 0.02
        m = torch.rand(shape, generator=g, device="cuda:0") < 0.01
        w[m] *= 50
        return w.view(torch.uint8).reshape(-1)
    if kind == "fp4":          # two near-uniform FP4 (e2m1) codes per byte (config 5 weights)
        return torch.randint(0, 256, shape, generator=g, device="cuda:0", dtype=torch.uint8).reshape(-1)
    if kind == "e8m0":         # E8M0 block scales: round(N(-6, 1.5)) + 127 (config 5 scales)
        s = torch.round(torch.randn(shape, generator=g, device="cuda:0") * 1.5 - 6) + 127
        return s.clamp(0, 255).to(torch.uint8).reshape(-1)
    raise ValueError(kind)


HUF, RANS = 1, 3   # reference codec wire ids (crates/ptwm-core/src/codec.rs:7-9)
EXACT_ROUTE = "decode_exact (reference streams) + merge"
REF_CHUNK = 256 << 10   # the reference's default compression_chunk (python/ptwm/_config.py:151)

# Each config in the reference's own plane formats, by tensor kind: (codec per
# plane, chunk size or 0).  The c*_ref workloads are these payloads (GPU-encoded,
# byte-identical to the reference encoder) on the exact route, and every line's
# CPU baseline decodes them on this host.
REF_FORMATS = {
    "c1": {"w": ([HUF, HUF], 0)},
    "c2": {"fp32o": ([HUF, HUF, HUF, RANS], REF_CHUNK)},
    "c3_huf": {"fp8": ([HUF, HUF], 0)},
    "c3_rans": {"fp8": ([RANS, RANS], 0)},
    "c4": {"w": ([HUF, HUF], REF_CHUNK), "n": ([HUF, HUF], REF_CHUNK)},
    "c5": {"fp4": ([HUF, HUF], 0), "e8m0": ([HUF], 0)},
}
REF_LINES = ("c1_ref", "c2_ref", "c3_huf", "c3_rans", "c5_ref")
CPU_FORMAT = {"llama8b": "c4", "bf16_1k": "c1", "c1_ref": "c1", "fp32_4k": "c2", "c2_ref": "c2", "fp8": "c3_huf",
              "c3_huf": "c3_huf", "fp8@rans": "c3_rans", "c3_rans": "c3_rans", "mxfp4": "c5", "c5_ref": "c5"}


MIN_DISTINCT_BYTES = 1 << 30   # rotate inputs of smaller workloads (the MALL holds 256 MB)


def parse_workload(name: str):
    """"<workload>[@rans][+crc][+hash]" -> (workload, codec tag, options)."""
    base, *opts = name.split("+")
    if set(opts) - {"crc", "hash"}:
        raise SystemExit(f"unknown workload option in {name}")
    wl_name, _, codec_tag = base.partition("@")
    if codec_tag not in ("", "rans"):
        raise SystemExit(f"unknown codec tag in {base}")
    return wl_name, codec_tag, set(opts)


def build_workload(name: str, resident: bool = False, integrity: bool = False) -> Workload:
    """`name` is a workload below, optionally suffixed "@rans" (GPU-native
    planes coded with rans_ilv).  With `integrity`, every plane's CRC-32 and
    every tensor's XXH64 are computed (by the library's own entry points) and
    kept, so that plan variants with and without them can be measured on the
    same compressed bytes (`plan_bytes`).  A workload under 1 GiB is built in
    as many distinct replicas (other seeds) as make 1 GiB, and consecutive
    steps decode consecutive replicas, so that no step finds its inputs in
    the 256 MB Infinity Cache; `resident` builds one replica (cache-resident
    numbers)."""
    from ptwm_amd import plan

    name, codec_tag, _ = parse_workload(name)
    native = "rans_ilv" if codec_tag == "rans" else "huff_ilv"

    CH = {"w": plan.CHAIN_IEEE16_SPLIT2, "n": plan.CHAIN_IEEE16_SPLIT2, "fp8": plan.CHAIN_E4M3_NIBBLE,
          "fp32o": plan.CHAIN_IEEE32_SPLIT4, "fp4": plan.CHAIN_NIBBLE_SPLIT, "e8m0": plan.CHAIN_PASSTHROUGH}
    # reference formats: (per-plane codecs, chunk size) by spec kind; None = the GPU-native codec
    ref = None
    exact = EXACT_ROUTE
    if name == "llama8b":
        specs = [(s, k) for _, s, k in llama8b_shapes()]
        desc = "config 4: Llama-3-8B-shaped bf16 model, 290 tensors, N(0,0.02) weights, norms 1+-0.01"
        kernel = "ilv_decode_kernel<1> (bf16 split2, fused decode+merge)"
    elif name == "fp8":
        specs = [((8192, 8192), "fp8")]
        desc = "config 3: float8_e4m3fn 8192x8192, per-row absmax N(0,1), E4M3 nibble split"
        kernel = "ilv_decode_kernel<3> (e4m3 nibble, fused decode+merge)"
    elif name == "bf16_1k":
        specs = [((1024, 1024), "w")]
        desc = "config 1: bf16 1024x1024 N(0,0.02), 2-plane split"
        kernel = "ilv_decode_kernel<1>"
    elif name == "fp32_4k":
        specs = [((4096, 4096), "fp32o")]
        desc = "config 2: fp32 4096x4096 N(0,0.02) + 1% x50 outliers, 4-plane split"
        kernel = "ilv_decode_kernel<2>"
    elif name == "bf16_1g":
        specs = [((32768, 16384), "w")]
        desc = "one bf16 32768x16384 N(0,0.02) tensor (1 GiB, config 4 distribution) for counter runs"
        kernel = "ilv_decode_kernel<1>"
    elif name == "mxfp4":
        specs = [((14336, 2048), "fp4"), ((14336, 128), "e8m0")]
        desc = "config 5: MXFP4 weights 14336x2048 (nibble split) + E8M0 scales 14336x128 (byte plane)"
        kernel = "ilv_decode_kernel<0x156> (two-chain launch: nibble split 5 + passthrough 6)"
    # the configs in the reference's own plane formats (GPU-encoded, byte-identical
    # to the reference encoder), decoded by the exact route
    elif name == "c1_ref":
        specs = [((1024, 1024), "w")]
        ref = REF_FORMATS["c1"]
        desc = "config 1 in reference format: bf16 1024x1024, Huffman on each plane"
        kernel = exact
    elif name == "c2_ref":
        specs = [((4096, 4096), "fp32o")]
        ref = REF_FORMATS["c2"]
        desc = "config 2 in reference format: fp32 4096x4096 + outliers, rANS exponent, Huffman mantissas, 256 KiB chunks"
        kernel = exact
    elif name == "c3_huf":
        specs = [((8192, 8192), "fp8")]
        ref = REF_FORMATS["c3_huf"]
        desc = "config 3 in reference format: e4m3 8192x8192, Huffman on both nibble planes"
        kernel = exact
    elif name == "c3_rans":
        specs = [((8192, 8192), "fp8")]
        ref = REF_FORMATS["c3_rans"]
        desc = "config 3 in reference format: e4m3 8192x8192, rANS on both nibble planes (unchunked)"
        kernel = exact
    elif name == "c5_ref":
        specs = [((14336, 2048), "fp4"), ((14336, 128), "e8m0")]
        ref = REF_FORMATS["c5"]
        desc = "config 5 in reference format: MXFP4 weights (Huffman nibble planes) + E8M0 scales (Huffman)"
        kernel = exact
    else:
        raise SystemExit(f"unknown workload {name}")
    if native == "rans_ilv" and ref is None:
        desc += ", planes coded with rans_ilv (GPU-native interleaved rANS)"
        kernel = kernel.replace("ilv_decode_kernel", "rilv_decode_kernel")
    if resident:
        n_rep = 1
    else:
        one = sum(int(np_prod(shape)) for shape, _ in specs)
        n_rep = max(1, -(-MIN_DISTINCT_BYTES // max(one, 1)))
    reps = [build_replica(desc, specs, CH, ref, native, integrity, r) for r in range(n_rep)]
    wl = reps[0]
    wl.replicas = reps
    wl.kernel = kernel
    wl.encode_gbs = sum(r.restored for r in reps) / sum(r.enc_s for r in reps) / 1e9
    wl.comp_bytes = round(sum(r.comp_bytes for r in reps) / n_rep)
    log(f"[bench] {n_rep} replica(s) of {wl.restored / 2**30:.3f} GiB; encoded at {wl.encode_gbs:.1f} GB/s input, "
        f"ratio {wl.comp_bytes / wl.restored:.4f}")
    return wl


def kernel_label(wl, crc: bool) -> str:
    """The dominant kernel's name for a plan variant: huff_ilv kernels carry a
    second template argument, plane CRC-32 computed in the decode (bf16, fp32
    and passthrough chains)."""
    k = wl.kernel
    if k == EXACT_ROUTE or k.startswith("rilv"):
        return k
    fused = crc and any(t.chain in (1, 2, 6) for t in wl.plans)
    k = re.sub(r"<(\d|0x[0-9a-f]+)>", lambda m: f"<{m.group(1)}, {'true' if fused else 'false'}>", k)
    return k + (" + plane CRC-32 fused" if fused else "")


def np_prod(shape):
    n = 1
    for d in shape:
        n *= d
    return n


def plan_bytes(rep, crc: bool, hsh: bool) -> bytes:
    """The replica's PTMD plan with or without plane CRC-32 and tensor XXH64."""
    import copy

    from ptwm_amd.plan import encode_plan

    plans = copy.deepcopy(rep.plans)
    for t in plans:
        if not hsh:
            t.xxh64 = None
        for p in t.planes:
            if not crc:
                p.crc32 = None
    return encode_plan(plans)


def build_replica(desc, specs, CH, ref, native, integrity, rep) -> Workload:
    import torch

    from ptwm_amd import api, plan

    wl = Workload(desc)
    wl.kinds = [kind for _, kind in specs]
    if ref is not None:
        wl.codec = "reference Huffman / rANS plane payloads (exact route)"
    elif native == "rans_ilv":
        wl.codec = "rans_ilv (GPU-native interleaved rANS, packed-nibble and stored forms) + Identity"
    else:
        wl.codec = "huff_ilv (GPU-native interleaved Huffman, packed-nibble and stored forms) + Identity"
    tensors = []
    total_raw = 0
    for i, (shape, kind) in enumerate(specs):
        raw = gen_tensor(kind, shape, 1000 + i + 7919 * rep)
        tensors.append((raw, CH[kind], ref[kind] if ref else None))
        total_raw += raw.numel()
    if rep == 0:
        log(f"[bench] generated {len(tensors)} tensors, {total_raw / 2**30:.2f} GiB")
    # encode every tensor with the library's GPU encoder into one blob
    cap = total_raw + 65536 * len(tensors) + (1 << 20)
    blob = torch.empty(cap, dtype=torch.uint8, device="cuda:0")
    off = 0
    out_off = 0
    plans = []
    torch.cuda.synchronize()   # the generators' kernels are not part of the encode
    if rep == 0:
        # one untimed call: the encoder's scratch buffers are allocated once per process
        if ref is None:
            api.encode_tensors_cuda([(chain, raw) for raw, chain, _ in tensors], blob, 0, codec=native)
        else:
            for raw, chain, rf in tensors:
                api.encode_tensor_ref_cuda(chain, rf[0], rf[1], raw, blob, 0)
        torch.cuda.synchronize()
    t0 = time.perf_counter()
    if ref is None:
        # GPU-native codecs: every tensor in one batched encoder call; the
        # median of three calls (the first warm call in a process has run
        # well below the rest)
        times = []
        for _ in range(3 if rep == 0 else 1):
            t0 = time.perf_counter()
            used, st = api.encode_tensors_cuda([(chain, raw) for raw, chain, _ in tensors], blob, 0, codec=native)
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t0)
        enc_s = sorted(times)[len(times) // 2]
        plans = plan.decode_plan(st)
        off = (used + 255) // 256 * 256
        out_off = plans[-1].out_offset + plans[-1].out_len if plans else 0
        out_off = (out_off + 255) // 256 * 256
    else:
        for raw, chain, rf in tensors:
            used, st = api.encode_tensor_ref_cuda(chain, rf[0], rf[1], raw, blob[off:], 0)
            t = plan.decode_plan(st)[0]
            t.out_offset = out_off
            for p in t.planes:
                p.payload_offset += off
            plans.append(t)
            off = (off + used + 255) // 256 * 256
            out_off = (out_off + raw.numel() + 255) // 256 * 256
        torch.cuda.synchronize()
        enc_s = time.perf_counter() - t0
    if integrity:
        for (raw, chain, _), t in zip(tensors, plans):
            for p, c in zip(t.planes, api.plane_crc32_cuda(chain, raw, 0)):
                p.crc32 = c
            t.xxh64 = api.xxh64_cuda(raw, 0)
    wl.tensors = tensors
    wl.blob = blob[:off]
    wl.plans = plans
    wl.plan_bytes = plan_bytes(wl, False, False)
    wl.out_len = out_off
    wl.restored = total_raw
    wl.comp_bytes = sum(p.payload_len for t in plans for p in t.planes)
    wl.enc_s = enc_s
    return wl


def verify(wl, out) -> bool:
    import torch

    for raw, t in zip((r for r, _, _ in wl.tensors), wl.plans):
        if not torch.equal(out[t.out_offset: t.out_offset + raw.numel()], raw):
            return False
    return True


def measure(wl, steps, warmup, crc=False, hsh=False):
    """Time `steps` decodes of the workload's plan variant (CRC-32 / XXH64
    verified or not) after `warmup` (at least one per replica), every
    restored byte checked after the warmup and after the timed steps.
    Returns (ms per step, dominant-kernel ms per step from HIP events)."""
    import torch

    from ptwm_amd import api, ids
    from ptwm_amd._native import lib

    L = lib()
    reps = wl.replicas
    plans = [plan_bytes(r, crc, hsh) for r in reps]
    outs = [torch.empty(r.out_len, dtype=torch.uint8, device="cuda:0") for r in reps]
    cur = [0]

    def step():
        k = cur[0] % len(reps)
        cur[0] += 1
        return api.hardware_backend_dispatch_decode_cuda(ids.HARDWARE_BACKEND_LABEL, ids.DECODE_PLAN_LABEL,
                                                         plans[k], reps[k].blob, outs[k], 0)

    def check(n, when):
        for r, o in list(zip(reps, outs))[:n]:
            if not verify(r, o):
                raise SystemExit(f"decode mismatch on {wl.name}{when}")

    for _ in range(max(warmup, len(reps))):
        step()
    torch.cuda.synchronize()
    check(len(reps), "")
    for o in outs:
        o.zero_()
    torch.cuda.synchronize()
    cur[0] = 0
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    # the replicas the timed steps decoded were zeroed before them
    check(min(steps, len(reps)), " (timed steps)")
    ms_step = (t1 - t0) * 1e3 / steps
    # kernel durations: HIP events around the decode kernels on the
    # library stream, in separate (untimed) steps so the events do not
    # add to the whole-call time above
    L.ptwm_mi355x_set_profiling(0, 1)
    ms = (C.c_float * 3)()
    kern = []
    for _ in range(min(steps, 5) if hsh else steps):
        step()
        L.ptwm_mi355x_last_kernel_ms(0, ms)
        # [0]: entropy decode (fused with the merge on the huff_ilv route),
        # [2]: every kernel of the call (exact route: decode + merge)
        kern.append(ms[2] if wl.kernel == EXACT_ROUTE else ms[0])
    L.ptwm_mi355x_set_profiling(0, 0)
    return ms_step, sum(kern) / len(kern)


def secondary_line(wl, ms, kms, crc=False, hsh=False):
    return {"restored_gbs": round(wl.restored / (ms * 1e-3) / 1e9, 1),
            "ms_per_step": round(ms, 4),
            "kernel_gbs_restored": round(wl.restored / (kms * 1e-3) / 1e9, 1),
            "kernel_gbs_traffic": round((wl.restored + wl.comp_bytes) / (kms * 1e-3) / 1e9, 1),
            "kernel": kernel_label(wl, crc),
            "ratio": round(wl.comp_bytes / wl.restored, 4), "encode_gbs": round(wl.encode_gbs, 1),
            "replicas": len(wl.replicas),
            "verified": "plane CRC-32 and tensor XXH64" if hsh else "plane CRC-32" if crc else "none",
            "description": wl.name}



def zstd_line(steps, with_cpu=True):
    """Zstd plane payloads at scale (codec 0x0004, zstd_device.hip): the bytes
    of a bf16 16384 x 32768 N(0, 0.02) tensor (1 GiB) as one passthrough
    plane in 256 KiB chunk frames ([version][state length 0][frame], as
    compressor.rs:316-381 writes chunked planes), each frame written by the
    image's libzstd at level 3 (the reference's Zstd codec calls libzstd at
    level 3, codecs/zstd.rs).  Every chunk is one wavefront's serial frame
    decode; the restored bytes are checked against the tensor after the
    timed steps.  CPU baseline: the oracle's RFC 8878 restatement decoding a
    sample of the same frames over 16 threads (and at one), with libzstd's
    own ZSTD_decompress on the same frames reported beside it."""
    import ctypes as C
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np
    import torch

    from ptwm_amd import api, ids, plan

    z = C.CDLL("libzstd.so.1")
    z.ZSTD_compressBound.argtypes = [C.c_size_t]
    z.ZSTD_compressBound.restype = C.c_size_t
    z.ZSTD_compress.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t, C.c_int]
    z.ZSTD_compress.restype = C.c_size_t
    z.ZSTD_decompress.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t]
    z.ZSTD_decompress.restype = C.c_size_t
    z.ZSTD_isError.argtypes = [C.c_size_t]
    z.ZSTD_isError.restype = C.c_uint
    g = torch.Generator(device="cuda:0").manual_seed(90)
    t = (torch.randn(16384, 32768, generator=g, device="cuda:0") * 0.02).to(torch.bfloat16)
    dev_raw = t.view(torch.uint8).reshape(-1)
    raw = dev_raw.cpu().numpy()
    n, CH = raw.size, 256 << 10
    t0 = time.perf_counter()
    frames = []
    for a in range(0, n, CH):
        part = np.ascontiguousarray(raw[a:a + CH])
        cap = z.ZSTD_compressBound(part.size)
        buf = np.empty(cap, np.uint8)
        r = z.ZSTD_compress(buf.ctypes.data, cap, part.ctypes.data, part.size, 3)
        if z.ZSTD_isError(r):
            raise SystemExit("libzstd compress failed")
        frames.append(buf[:r].tobytes())
    enc_s = time.perf_counter() - t0
    body, ents = bytearray(), []
    for k, f in enumerate(frames):
        ents.append((len(body), min(CH, n - k * CH)))
        body += b"\x00\x00\x00\x00\x00" + f
    pp = plan.PlanePlan(ids.CODEC_ZSTD, 0, len(body), n, ents)
    state = plan.encode_plan([plan.TensorPlan(plan.CHAIN_PASSTHROUGH, 0, n, [pp])])
    src = torch.from_numpy(np.frombuffer(bytes(body), np.uint8).copy()).to("cuda:0")
    out = torch.empty(n, dtype=torch.uint8, device="cuda:0")

    def step():
        return api.hardware_backend_dispatch_decode_cuda(ids.HARDWARE_BACKEND_LABEL, ids.DECODE_PLAN_LABEL, state,
                                                         src, out, 0)

    step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / steps * 1e3
    if not torch.equal(out, dev_raw):
        raise SystemExit("zstd: restored bytes differ from the tensor")
    line = {"restored_gbs": round(n / (ms * 1e-3) / 1e9, 2), "ms_per_step": round(ms, 3),
            "kernel": "zstd_decode_kernel (one wavefront per 256 KiB chunk frame)",
            "ratio": round(len(body) / n, 4), "frames": len(frames),
            "encode": f"libzstd level 3 on the host, {n / enc_s / 1e9:.2f} GB/s (input to the bench, not measured)",
            "description": "bf16 16384x32768 N(0,0.02) bytes (1 GiB) as one passthrough plane, 256 KiB Zstd chunk frames"}
    if with_cpu:
        import oracle as O

        sample = list(range(0, len(frames), max(1, len(frames) // 32)))[:32]
        sizes = [ents[k][1] for k in sample]
        nbytes = sum(sizes)
        for k in sample[:4]:  # the restatement decodes the same frames bit-exactly
            if O.zstd_decompress(frames[k], sizes[sample.index(k)]) != raw[k * CH:k * CH + sizes[sample.index(k)]].tobytes():
                raise SystemExit("zstd: CPU restatement differs")
        outs = [np.empty(sz, np.uint8) for sz in sizes]
        srcs = [np.frombuffer(frames[k], np.uint8) for k in sample]

        def port(i):
            O.zstd_decompress(frames[sample[i]], sizes[i])

        def libz(i):
            r = z.ZSTD_decompress(outs[i].ctypes.data, sizes[i], srcs[i].ctypes.data, srcs[i].size)
            if z.ZSTD_isError(r):
                raise SystemExit("libzstd decompress failed")

        def rate(fn, nthreads, budget=1.0):
            with ThreadPoolExecutor(nthreads) as ex:
                t0, reps = time.perf_counter(), 0
                while True:
                    list(ex.map(fn, range(len(sample))))
                    reps += 1
                    if time.perf_counter() - t0 > budget:
                        break
                return round(nbytes * reps / (time.perf_counter() - t0) / 1e9, 3)

        threads = min(16, os.cpu_count() or 1)
        line["cpu_baseline"] = {"value": rate(port, threads), "unit": "GB/s", "cores": threads, "kind": "port",
                                "value_1_thread": rate(port, 1),
                                "libzstd_gbs": rate(libz, threads), "libzstd_gbs_1_thread": rate(libz, 1),
                                "sample": f"{len(sample)} of the {len(frames)} frames ({nbytes / 2**20:.0f} MiB), "
                                          "oracle/zstd_oracle.c; libzstd ZSTD_decompress on the same frames"}
    return line

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="llama8b+crc",
                    help="<workload>[@rans][+crc][+hash]: the headline decode (default: config 4, plane "
                         "CRC-32 verified inside the timed region)")
    ap.add_argument("--extra", default="fp8,fp8@rans,mxfp4,bf16_1k,fp32_4k,c1_ref,c2_ref,c3_huf,c3_rans,c5_ref,zstd",
                    help="comma list of secondary workloads reported in config")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--resident", action="store_true",
                    help="one replica of a workload under 1 GiB (inputs may stay in the Infinity Cache)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a 1 GiB device copy (known bytes) to scale FETCH_SIZE/WRITE_SIZE counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; --gpus above 1 is not part of it",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    import torch

    if args.copy_calibration:
        a = torch.ones(1 << 30, dtype=torch.uint8, device="cuda:0")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        del a, b
        log("[bench] calibration copy: 3 x 1 GiB device-to-device")
    log(f"[bench] workload {args.workload}")
    _, _, opts = parse_workload(args.workload)
    crc, hsh = "crc" in opts, "hash" in opts
    wl = build_workload(args.workload, args.resident, integrity=bool(opts) or args.workload == "llama8b")
    ms_step, kms = measure(wl, args.steps, args.warmup, crc, hsh)
    value = wl.restored / (ms_step * 1e-3) / 1e9
    traffic = wl.comp_bytes + wl.restored
    achieved = traffic / (kms * 1e-3) / 1e9
    verified = "plane CRC-32 and tensor XXH64" if hsh else "plane CRC-32" if crc else "none"
    primary = {"workload": args.workload, "description": wl.name, "verified_in_timed_region": verified,
               "restored_bytes": wl.restored, "compressed_bytes": wl.comp_bytes,
               "ratio": round(wl.comp_bytes / wl.restored, 4), "encode_gbs": round(wl.encode_gbs, 1),
               "hbm_frac_of_peak": round(value / HBM_PEAK_GBS, 4), "codec": wl.codec,
               "replicas": len(wl.replicas), "distinct_input_bytes": sum(r.comp_bytes for r in wl.replicas)}
    kernel_name = kernel_label(wl, crc)
    log(f"[bench] {ms_step:.3f} ms/step, kernel {kms:.3f} ms, {value:.1f} GB/s restored ({verified} verified)")
    extras = {}
    base = args.workload.split("+")[0]
    if wl.plans and wl.plans[0].xxh64 is not None:
        # the same compressed bytes: without any verification, and with the
        # tensor XXH64 as well (reported in its own field)
        if crc or hsh:
            m2, k2 = measure(wl, args.steps, 1)
            extras[base] = secondary_line(wl, m2, k2)
            log(f"[bench] {base} without verification: {m2:.3f} ms/step")
        if not hsh:
            m3, k3 = measure(wl, 3, 1, True, True)
            primary["hash_verified"] = secondary_line(wl, m3, k3, True, True)
            log(f"[bench] {base} with CRC-32 + XXH64: {m3:.3f} ms/step")
    cpu = None
    if not args.no_cpu_baseline and base in CPU_FORMAT:
        # config 4: the tensors of layer 0 (a bounded sample of the same model)
        sample = [i for i, t in enumerate(llama8b_shapes()) if ".layers.0." in t[0]] if base == "llama8b" else None
        cpu = cpu_line(wl, base, sample, budget_s=3.0)
        log(f"[bench] CPU restatement: {cpu['value']} GB/s at {cpu['cores']} threads, {cpu['value_1_thread']} at 1")
    for name in [x for x in args.extra.split(",") if x and x != args.workload]:
        del wl
        gc.collect()
        torch.cuda.empty_cache()
        if name == "zstd":
            wl = None
            extras[name] = zstd_line(max(3, args.steps // 2), not args.no_cpu_baseline)
            log(f"[bench] zstd: {extras[name]['restored_gbs']} GB/s restored"
                + (f", CPU {extras[name]['cpu_baseline']['value']} GB/s (libzstd "
                   f"{extras[name]['cpu_baseline']['libzstd_gbs']})" if "cpu_baseline" in extras[name] else ""))
            continue
        slow = name == "c3_rans"   # four serial rANS chains per 64 MiB plane: seconds per step
        wl = build_workload(name, args.resident or slow)
        m2, k2 = measure(wl, 1 if slow else max(3, args.steps), 0 if slow else 1)
        extras[name] = secondary_line(wl, m2, k2)
        if not args.no_cpu_baseline:
            extras[name]["cpu_baseline"] = cpu_line(wl, name, budget_s=1.0)
        log(f"[bench] {name}: {extras[name]['restored_gbs']} GB/s restored"
            + (f", CPU {extras[name]['cpu_baseline']['value']} GB/s" if "cpu_baseline" in extras[name] else ""))
    primary["secondary"] = extras
    traffic_meas, traffic_src = measured_traffic(args.workload)
    ceil = hbm_ceilings()
    # the workload's bound from those ceilings: its R restored bytes must be
    # written (write ceiling) and its C + R bytes moved (copy ceiling)
    t_min = max(primary["restored_bytes"] / (ceil["write_gbs"] * 1e9),
                (primary["restored_bytes"] + primary["compressed_bytes"]) / (ceil["copy_gbs"] * 1e9))
    ceil["restored_gbs_bound"] = round(primary["restored_bytes"] / t_min / 1e9, 1)
    ceil["kernel_frac_of_bound"] = round(t_min / (kms * 1e-3), 4)
    res = {
        "metric": "decode GB/s (restored bytes) per MI355X",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic (seeded torch generators on device)",
        "config": primary,
        "roofline": {"bound": "hbm", "kernel": kernel_name, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "kernel_ms": round(kms, 4),
                     "traffic": traffic_meas, "traffic_source": traffic_src, "ceilings": ceil},
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)


def hbm_ceilings():
    """Practical HBM rates of this device, measured in the same run: a 2 GiB
    device copy (reads + writes) and a 2 GiB fill (writes only), torch's own
    kernels, best of 5."""
    import torch

    n = 2 << 30
    a = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    b = torch.empty_like(a)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def best(fn):
        ms = []
        for _ in range(5):
            e0.record()
            fn()
            e1.record()
            e1.synchronize()
            ms.append(e0.elapsed_time(e1))
        return min(ms)

    copy_ms = best(lambda: b.copy_(a))
    fill_ms = best(lambda: b.fill_(7))
    del a, b
    torch.cuda.empty_cache()
    return {"copy_gbs": round(2 * n / (copy_ms * 1e-3) / 1e9, 1), "write_gbs": round(n / (fill_ms * 1e-3) / 1e9, 1),
            "source": "torch copy_ / fill_ of 2 GiB on this device, same run"}


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_line(wl, name: str, sample=None, budget_s: float = 1.5):
    """The oracle's C restatement of the reference CPU codec, timed on this
    host, on this line's own input: replica 0's tensors (or the `sample` of
    them), copied to host memory, in the config's reference plane format
    (REF_FORMATS).  Encode (forward chain, then per plane Huffman or rANS,
    chunk frames and table) and decode (chunks of every plane over the
    threads as container.rs:1773,1996 run them, then the inverse chain),
    each at min(16, nproc) threads and at one thread, passes repeated for
    about `budget_s`.  For the c*_ref lines the CPU-encoded payloads are
    checked equal to the GPU-encoded ones that line decodes, so both read
    the same compressed bytes; every CPU decode is checked bit-exact."""
    import oracle as O

    fmt = REF_FORMATS[CPU_FORMAT[name]]
    rep = wl.replicas[0]
    idx = list(range(len(rep.tensors))) if sample is None else list(sample)
    raws, items = [], []
    for i in idx:
        raw, chain, _ = rep.tensors[i]
        codecs, chunk = fmt[rep.kinds[i]]
        h = raw.cpu().numpy()
        raws.append(h)
        items.append((chain, h, [(c, chunk) for c in codecs]))
    threads = min(16, os.cpu_count() or 1)
    enc = O.PlaneBatchEncoder(items)
    enc.encode(threads)
    planes = enc.planes()
    if name in REF_LINES:
        blob = rep.blob.cpu().numpy()
        k = 0
        for i in idx:
            for p in rep.plans[i].planes:
                gpu = blob[p.payload_offset: p.payload_offset + p.payload_len].tobytes()
                if planes[k][0] != gpu:
                    raise SystemExit(f"{name}: GPU-encoded payload differs from the CPU restatement's (plane {k})")
                k += 1
    batch, k = [], 0
    for (chain, h, pl) in items:
        batch.append((chain, h.size, [(c, *planes[k + j]) for j, (c, _) in enumerate(pl)]))
        k += len(pl)
    dec = O.PlaneBatch(batch)
    dec.decode(threads)
    for n, h in enumerate(raws):
        if dec.outs[n][: h.size].tobytes() != h.tobytes():
            raise SystemExit(f"{name}: CPU restatement round trip differs")
    nbytes = dec.restored
    comp = sum(len(p) for p, _ in planes)

    def rate(fn, nthreads):
        t0 = time.perf_counter()
        reps = 0
        while True:
            fn(nthreads)
            reps += 1
            if time.perf_counter() - t0 > budget_s:
                break
        return nbytes * reps / (time.perf_counter() - t0) / 1e9, reps

    dn, rn = rate(dec.decode, threads)
    d1, r1 = rate(dec.decode, 1)
    en, _ = rate(enc.encode, threads)
    e1, _ = rate(enc.encode, 1)
    fmt_txt = "; ".join(f"{kd}: {'/'.join('rANS' if c == RANS else 'Huffman' for c in cs)}"
                        f"{f' in {ch >> 10} KiB chunks' if ch else ''}" for kd, (cs, ch) in fmt.items())
    return {"value": round(dn, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "value_1_thread": round(d1, 3), "encode_gbs": round(en, 3), "encode_gbs_1_thread": round(e1, 3),
            "nproc": os.cpu_count(), "cpu_model": cpu_model(),
            "sample": f"{len(idx)} tensor(s), {nbytes / 2**20:.1f} MiB restored, ratio {comp / nbytes:.4f}, "
                      f"reference format ({fmt_txt}); {rn} decode passes at {threads} threads, {r1} at 1; "
                      "oracle C restatement, chunks over threads, no CRC-32 / XXH64"}


if __name__ == "__main__":
    main()
