// abi.hip -- extern "C" entry points of libptwm_mi355x.so.
//
// The reference's native extension ABI (crates/ptwm-core/src/flavor/
// native.rs:62-197) plus this library's additions; declarations and the
// contract of every symbol are in include/ptwm_mi355x.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <cstring>

#include "../../include/ptwm_mi355x.h"
#include "decode_sync.h"
#include "ilv_host.h"
#include "integrity.h"
#include "plane_ops.h"
#include "ref_encode.h"
#include "runtime.h"

namespace ptwm {
namespace {

// Built-in canonical ids: blake3([0xBB;32] || 0 || name || 0 || version)
// (extension/id.rs:21-30, extension/mod.rs:36, builtins.rs:18-27).  Both the
// current (1.1.0) and the 1.0.0 derivations are accepted, as readers map
// older ids to the current ones (builtins.rs:20-26).
struct KnownId {
  const char* hex;
  uint32_t codec;
};
constexpr KnownId kBuiltinIds[] = {
    {"fc2dea1265e3394c57c2df3b868b732ccaa1ee876bd4b1ce27d38f842c6112b5", kCodecIdentity},  // identity@1.1.0
    {"614155b5a8c9efb689219bcca3cbf7855e29d3023208ce61cca7a36849248e33", kCodecHuffman},   // huffman@1.1.0
    {"39c875ef9793a9c5ebe199116debac4c9d5388b8b7cf2fe6b575845f0ca1624e", kCodecRans},      // rans@1.1.0
    {"eb31edfe6fd156b309010ca750571766fc8ae6e4056bc2b4a228679922edea30", kCodecIdentity},  // identity@1.0.0
    {"571e8fae548f0db5faa961fb65ba5ea2443bdb1e95dac04fbf1d5d97228ec945", kCodecHuffman},   // huffman@1.0.0
    {"87c8ca053fbd0646c07d18da4d0396a92550eb6d44bcd4e461538902874d4bc7", kCodecRans},      // rans@1.0.0
    {"e4868545e7b22282695972441494e70569ab27595d19349114e852125d96daa4", kCodecTans},      // tans@1.1.0
    {"ee06c9c76d008d4cfd5dca6289485aecc5328a88b035b6bc7583eb88d218fd8f", kCodecTans},      // tans@1.0.0
    // this extension: blake3([0;32] || 0 || "io.ptwm.mi355x.plane_codec" || 0 || "0.1.0")
    {"cfd8cc03483eb4a43cdddb4b3cbf95b32e0a3f0e17e5ec85a0b52de04e8caf04", kCodecHuffIlv},
    // blake3([0;32] || 0 || "io.ptwm.mi355x.plane_codec.rans" || 0 || "0.1.0")
    {"968f8be9f06b14b33fcd066622493f1101954d074c25d63e78380d33708fe1f5", kCodecRansIlv},
};
// blake3([0;32] || 0 || "io.ptwm.mi355x.hardware_backend" || 0 || "0.1.0")
constexpr const char* kBackendIdHex = "a432dc02f57030b41a3660762bbcec5668cde8abbc807999d56ca0a3304d39cf";
// blake3([0;32] || 0 || "io.ptwm.mi355x.decode_plan" || 0 || "0.1.0")
constexpr const char* kPlanIdHex = "1b0e48b156b01d0d733a5aa62a90bcbde34945ff024d8d8e56cb714a48c6e770";
constexpr const char* kOwnCodecIdHex = "cfd8cc03483eb4a43cdddb4b3cbf95b32e0a3f0e17e5ec85a0b52de04e8caf04";
constexpr const char* kRansCodecIdHex = "968f8be9f06b14b33fcd066622493f1101954d074c25d63e78380d33708fe1f5";

bool hex_eq(const char* hex, const uint8_t* id) {
  for (int i = 0; i < 32; ++i) {
    auto nib = [](char c) -> int { return c <= '9' ? c - '0' : c - 'a' + 10; };
    int v = (nib(hex[2 * i]) << 4) | nib(hex[2 * i + 1]);
    if (v != id[i]) return false;
  }
  return true;
}

void hex_to(const char* hex, uint8_t* out) {
  for (int i = 0; i < 32; ++i) {
    auto nib = [](char c) -> int { return c <= '9' ? c - '0' : c - 'a' + 10; };
    out[i] = (uint8_t)((nib(hex[2 * i]) << 4) | nib(hex[2 * i + 1]));
  }
}

// Resolve a codec id to a wire id; returns false if unknown.
bool lookup_codec(const uint8_t* id, size_t len, uint32_t& codec) {
  if (!id || len != 32) return false;
  for (const KnownId& k : kBuiltinIds)
    if (hex_eq(k.hex, id)) {
      codec = k.codec;
      return true;
    }
  return false;
}

// RAII: lock the device context, make its device current, restore after.
// Stream the calling thread asked the library to run on, per device
// (ptwm_mi355x_use_stream); calls without one use the library's own stream.
struct ThreadStream {
  uint32_t dev = 0;
  uint64_t stream = 0;
  bool set = false;
};
thread_local ThreadStream t_stream;

struct DeviceScope {
  DevCtx* ctx;
  std::unique_lock<std::mutex> lk;
  int prev = -1;
  bool ok = false;
  // create: make the device's context on first use (every entry point but
  // the allocation-free decode, which only takes an existing one)
  explicit DeviceScope(uint32_t ord, bool create = true) : ctx(create ? get_ctx(ord) : find_ctx(ord)) {
    if (!ctx) return;
    lk = std::unique_lock<std::mutex>(ctx->mu);
    ctx->stream = t_stream.set && t_stream.dev == ord ? reinterpret_cast<hipStream_t>(t_stream.stream) : ctx->own_stream;
    (void)hipGetDevice(&prev);
    ok = hipSetDevice(ctx->dev) == hipSuccess;
  }
  ~DeviceScope() {
    if (ctx && prev >= 0) (void)hipSetDevice(prev);
  }
};

int64_t decode_one_payload(DevCtx& ctx, uint32_t codec, uint64_t in_dev, size_t in_len, uint64_t out_dev,
                           size_t out_cap) {
  uint64_t expected = 0;
  if (codec == kCodecIdentity) {
    expected = in_len;
  } else if (codec == kCodecHuffman || codec == kCodecRans || codec == kCodecTans) {
    if (in_len == 0) return kInvalidInput;
    PTWM_HIP_TRY(ctx.h_small.ensure(64));
    uint8_t* hdr = static_cast<uint8_t*>(ctx.h_small.ptr);
    size_t n = in_len < 5 ? in_len : 5;
    PTWM_HIP_TRY(hipMemcpyAsync(hdr, reinterpret_cast<const void*>(in_dev), n, hipMemcpyDeviceToHost, ctx.stream));
    PTWM_HIP_TRY(hipStreamSynchronize(ctx.stream));
    if (hdr[0] == 0) {
      expected = in_len - 1;
    } else if (hdr[0] == 1 && in_len >= 5) {
      expected = (uint64_t)hdr[1] | ((uint64_t)hdr[2] << 8) | ((uint64_t)hdr[3] << 16) | ((uint64_t)hdr[4] << 24);
    } else {
      return kInvalidInput;
    }
  } else {
    return kUnsupported;
  }
  if (expected > out_cap) return kBufferTooSmall;
  if (expected == 0 && codec == kCodecIdentity) return 0;
  PTWM_HIP_TRY(ctx.h_jobs.ensure(sizeof(DecodeJob)));
  DecodeJob* J = static_cast<DecodeJob*>(ctx.h_jobs.ptr);
  std::memset(J, 0, sizeof(*J));
  J->src = in_dev;
  J->src_len = in_len;
  J->dst = out_dev;
  J->dst_len = expected;
  J->codec = codec;
  J->framed = 0;
  const int64_t rc = decode_jobs(ctx, J, 1);
  if (rc != kOk) return rc;
  if (*static_cast<uint32_t*>(ctx.h_status.ptr) != kStOk) return kInvalidInput;
  return (int64_t)expected;
}

// One huff_ilv or rans_ilv payload -> plane bytes (fused kernel,
// passthrough chain).
int64_t ilv_decode_payload(DevCtx& ctx, uint64_t in_dev, size_t in_len, uint64_t out_dev, size_t out_cap,
                           uint32_t family = kFamilyHuff) {
  if (in_len == 0) return kInvalidInput;
  PTWM_HIP_TRY(ctx.h_small.ensure(64));
  uint8_t* hdr = static_cast<uint8_t*>(ctx.h_small.ptr);
  const size_t nh = in_len < 5 ? in_len : 5;
  PTWM_HIP_TRY(hipMemcpyAsync(hdr, reinterpret_cast<const void*>(in_dev), nh, hipMemcpyDeviceToHost, ctx.stream));
  PTWM_HIP_TRY(hipStreamSynchronize(ctx.stream));
  uint64_t expected;
  if (hdr[0] == 0) {
    expected = in_len - 1;
  } else if ((hdr[0] == 1 && in_len >= 5) || (hdr[0] == 2 && in_len >= kPackedHeadBytes)) {
    // coded (tag 1) and packed-nibble (tag 2) payloads carry n after the tag
    expected = (uint64_t)hdr[1] | ((uint64_t)hdr[2] << 8) | ((uint64_t)hdr[3] << 16) | ((uint64_t)hdr[4] << 24);
  } else {
    return kInvalidInput;
  }
  if (expected > out_cap) return kBufferTooSmall;
  if (expected == 0) return 0;
  if (hdr[0] == 0) {
    PTWM_HIP_TRY(launch_copy(reinterpret_cast<const uint8_t*>(in_dev + 1), reinterpret_cast<uint8_t*>(out_dev),
                             expected, ctx.stream));
    PTWM_HIP_TRY(hipStreamSynchronize(ctx.stream));
    return (int64_t)expected;
  }
  // the fused kernel stores 16-byte pieces: an output that is not 16-byte
  // aligned is decoded into aligned staging and copied
  const bool realign = (out_dev & 15u) != 0;
  if (realign) PTWM_HIP_TRY(ctx.stage_out.ensure(expected + 64));
  IlvTensor X{};
  X.out = realign ? reinterpret_cast<uint64_t>(ctx.stage_out.ptr) : out_dev;
  X.n = expected;
  X.chain = kChainPassthrough;
  X.n_planes = 1;
  X.planes[0].base = in_dev;
  X.planes[0].len = in_len;
  X.planes[0].coded = 1;
  X.family = family;
  X.crc_first = kIlvNoCrc;
  int64_t rc = ilv_decode_tensors(ctx, std::vector<IlvTensor>{X});
  if (rc != kOk) return rc;
  if (realign) {
    PTWM_HIP_TRY(hipMemcpyAsync(reinterpret_cast<void*>(out_dev), ctx.stage_out.ptr, expected,
                                hipMemcpyDeviceToDevice, ctx.stream));
    PTWM_HIP_TRY(hipStreamSynchronize(ctx.stream));
  }
  return (int64_t)expected;
}

// Host-buffer entry points stage through device memory on device 0.
constexpr uint32_t kHostDevice = 0;

static_assert(PTWM_MI355X_NOALLOC_SCRATCH_BYTES == kNoAllocScratchBytes, "allocation-free scratch size");
static_assert(PTWM_MI355X_NOALLOC_MAX_TENSORS == kNoAllocMaxTensors, "allocation-free tensor limit");
static_assert(PTWM_MI355X_NOALLOC_MAX_CRC_BLOCKS == kNoAllocMaxCrcBlocks, "allocation-free CRC block limit");

// The tensor-level decode's argument checks: the decode-plan id, the plan
// itself (parse_plan) and tensors that do not overlap in the output.
// *total: the restored bytes.
int64_t accept_plan(const uint8_t* state_ptr, size_t state_len, const uint8_t* codec_id_ptr, size_t codec_id_len,
                    uint64_t in_dev_ptr, size_t in_len, uint64_t out_dev_ptr, size_t out_len, Plan& plan,
                    uint64_t* total) {
  if (!codec_id_ptr || codec_id_len != 32 || !hex_eq(kPlanIdHex, codec_id_ptr)) return kUnsupported;
  int64_t rc = parse_plan(state_ptr, state_len, in_len, out_len, plan);
  if (rc != kOk) return rc;
  std::vector<std::pair<uint64_t, uint64_t>> spans;
  *total = 0;
  for (const PlanTensor& t : plan.tensors) {
    spans.emplace_back(t.out_offset, t.out_len);
    *total += t.out_len;
  }
  std::sort(spans.begin(), spans.end());
  for (size_t i = 1; i < spans.size(); ++i)
    if (spans[i - 1].first + spans[i - 1].second > spans[i].first) return kInvalidInput;
  if (*total && (!in_dev_ptr || !out_dev_ptr)) return kInvalidInput;
  return kOk;
}

}  // namespace
}  // namespace ptwm

using namespace ptwm;

extern "C" {

uint32_t ptwm_mi355x_abi_version(void) { return 1; }

int64_t ptwm_mi355x_canonical_id(uint32_t which, uint8_t* out32) {
  if (!out32) return kInvalidInput;
  const char* hex = which == 0   ? kOwnCodecIdHex
                    : which == 1 ? kBackendIdHex
                    : which == 2 ? kPlanIdHex
                    : which == 3 ? kRansCodecIdHex
                                 : nullptr;
  if (!hex) return kInvalidInput;
  hex_to(hex, out32);
  return 0;
}

uint64_t ptwm_plane_codec_v1_cuda_stream_handle(uint32_t device_ordinal) {
  DevCtx* c = get_ctx(device_ordinal);
  return c ? reinterpret_cast<uint64_t>(c->own_stream) : 0;
}

uint64_t ptwm_hardware_backend_v1_cuda_stream_handle(uint32_t device_ordinal) {
  return ptwm_plane_codec_v1_cuda_stream_handle(device_ordinal);
}

int64_t ptwm_plane_codec_v1_decode_cuda(uint8_t state_format_version, const uint8_t* state_ptr, size_t state_len,
                                        const uint8_t* codec_id_ptr, size_t codec_id_len, uint64_t in_dev_ptr,
                                        size_t in_len, uint64_t out_dev_ptr, size_t out_cap,
                                        uint32_t device_ordinal) {
  (void)state_format_version;
  (void)state_ptr;
  uint32_t codec = 0;
  if (!lookup_codec(codec_id_ptr, codec_id_len, codec)) return kUnsupported;
  if (state_len != 0) return kInvalidInput;  // none of these codecs carries state
  if ((in_len && !in_dev_ptr) || (out_cap && !out_dev_ptr)) return kInvalidInput;
  DeviceScope ds(device_ordinal);
  if (!ds.ok) return kInvalidInput;
  if (codec == kCodecHuffIlv) return ilv_decode_payload(*ds.ctx, in_dev_ptr, in_len, out_dev_ptr, out_cap);
  if (codec == kCodecRansIlv)
    return ilv_decode_payload(*ds.ctx, in_dev_ptr, in_len, out_dev_ptr, out_cap, kFamilyRans);
  return decode_one_payload(*ds.ctx, codec, in_dev_ptr, in_len, out_dev_ptr, out_cap);
}

int64_t ptwm_plane_codec_v1_encode_cuda(uint8_t state_format_version, const uint8_t* state_ptr, size_t state_len,
                                        const uint8_t* codec_id_ptr, size_t codec_id_len, uint64_t in_dev_ptr,
                                        size_t in_len, uint64_t out_dev_ptr, size_t out_cap, uint64_t* needed_out,
                                        uint32_t device_ordinal) {
  (void)state_format_version;
  (void)state_ptr;
  uint32_t codec = 0;
  if (!lookup_codec(codec_id_ptr, codec_id_len, codec)) return kUnsupported;
  if (state_len != 0) return kInvalidInput;
  if ((in_len && !in_dev_ptr) || (out_cap && !out_dev_ptr)) return kInvalidInput;
  if (codec == kCodecHuffman || codec == kCodecRans || codec == kCodecIdentity) {
    // the reference's payloads, byte-identical to its encoder
    DeviceScope ds(device_ordinal);
    if (!ds.ok) return kInvalidInput;
    if (codec == kCodecIdentity) {  // codecs/identity.rs: payload = plane
      if (in_len > out_cap) {
        if (needed_out) *needed_out = in_len;
        return kBufferTooSmall;
      }
      if (in_len) {
        PTWM_HIP_TRY(hipMemcpyAsync(reinterpret_cast<void*>(out_dev_ptr), reinterpret_cast<const void*>(in_dev_ptr),
                                    in_len, hipMemcpyDeviceToDevice, ds.ctx->stream));
        PTWM_HIP_TRY(hipStreamSynchronize(ds.ctx->stream));
      }
      return (int64_t)in_len;
    }
    RefEncoder enc;
    std::vector<uint64_t> len;
    int64_t rc = enc.plan(*ds.ctx, {RefJob{in_dev_ptr, in_len, codec}}, len);
    if (rc < 0) return rc;
    if (len[0] > out_cap) {
      if (needed_out) *needed_out = len[0];
      return kBufferTooSmall;
    }
    rc = enc.write(*ds.ctx, {out_dev_ptr});
    return rc < 0 ? rc : (int64_t)len[0];
  }
  if (codec != kCodecHuffIlv && codec != kCodecRansIlv) return kUnsupported;
  DeviceScope ds(device_ordinal);
  if (!ds.ok) return kInvalidInput;
  DevCtx& ctx = *ds.ctx;
  // the encoder reads dwordx4 and writes 4-byte words: a plane or an output
  // buffer at other alignments (a torch slice) goes through aligned staging
  uint64_t src = in_dev_ptr, dst = out_dev_ptr;
  if (in_len && (src & 15u)) {
    PTWM_HIP_TRY(ctx.stage_in.ensure(in_len + 16));
    PTWM_HIP_TRY(hipMemcpyAsync(ctx.stage_in.ptr, reinterpret_cast<const void*>(src), in_len,
                                hipMemcpyDeviceToDevice, ctx.stream));
    src = reinterpret_cast<uint64_t>(ctx.stage_in.ptr);
  }
  const bool restage = out_cap && (dst & 3u);
  if (restage) {
    PTWM_HIP_TRY(ctx.stage_out.ensure(out_cap + 16));
    dst = reinterpret_cast<uint64_t>(ctx.stage_out.ptr);
  }
  IlvEncResult r{};
  uint64_t needed = 0, n = in_len;
  int64_t rc = codec == kCodecHuffIlv ? ilv_encode_planes(ctx, &src, &n, 1, dst, out_cap, false, &r, &needed)
                                      : rilv_encode_planes(ctx, &src, &n, 1, dst, out_cap, false, &r, &needed);
  if (rc == kBufferTooSmall && needed_out) *needed_out = needed;
  if (rc < 0) return rc;
  if (restage && r.len) {
    PTWM_HIP_TRY(hipMemcpyAsync(reinterpret_cast<void*>(out_dev_ptr), ctx.stage_out.ptr, r.len,
                                hipMemcpyDeviceToDevice, ctx.stream));
    PTWM_HIP_TRY(hipStreamSynchronize(ctx.stream));
  }
  return (int64_t)r.len;
}

int64_t ptwm_hardware_backend_v1_dispatch_decode_cuda(uint8_t state_format_version, const uint8_t* state_ptr,
                                                      size_t state_len, const uint8_t* codec_id_ptr,
                                                      size_t codec_id_len, uint64_t in_dev_ptr, size_t in_len,
                                                      uint64_t out_dev_ptr, size_t out_len,
                                                      uint32_t device_ordinal) {
  (void)state_format_version;
  Plan plan;
  uint64_t total = 0;
  int64_t rc = accept_plan(state_ptr, state_len, codec_id_ptr, codec_id_len, in_dev_ptr, in_len, out_dev_ptr,
                           out_len, plan, &total);
  if (rc != kOk) return rc;
  DeviceScope ds(device_ordinal);
  if (!ds.ok) return kInvalidInput;
  rc = execute_plan(*ds.ctx, plan, in_dev_ptr, out_dev_ptr);
  return rc == kOk ? (int64_t)total : rc;
}

int64_t ptwm_mi355x_dispatch_decode_noalloc_cuda(uint8_t state_format_version, const uint8_t* state_ptr,
                                                 size_t state_len, const uint8_t* codec_id_ptr, size_t codec_id_len,
                                                 uint64_t in_dev_ptr, size_t in_len, uint64_t out_dev_ptr,
                                                 size_t out_len, uint32_t device_ordinal) {
  (void)state_format_version;
  Plan plan;
  uint64_t total = 0;
  int64_t rc = accept_plan(state_ptr, state_len, codec_id_ptr, codec_id_len, in_dev_ptr, in_len, out_dev_ptr,
                           out_len, plan, &total);
  if (rc != kOk) return rc;
  DeviceScope ds(device_ordinal, false);
  if (!ds.ctx) return kMissingCapability;  // ptwm_mi355x_device_init was not called for this device
  if (!ds.ok) return kInvalidInput;
  rc = execute_plan_noalloc(*ds.ctx, plan, in_dev_ptr, out_dev_ptr);
  return rc == kOk ? (int64_t)total : rc;
}

int64_t ptwm_plane_codec_v1_encode(const uint8_t* in, size_t in_len, uint8_t* out, size_t out_len) {
  if ((in_len && !in) || (out_len && !out)) return kInvalidInput;
  DeviceScope ds(kHostDevice);
  if (!ds.ok) return kMissingCapability;
  DevCtx& ctx = *ds.ctx;
  PTWM_HIP_TRY(ctx.stage_in.ensure(in_len + 16));
  const uint64_t bound = in_len + 1;  // stored size; the coded size is smaller or unused
  PTWM_HIP_TRY(ctx.stage_out.ensure(bound + 64));
  if (in_len) PTWM_HIP_TRY(hipMemcpyAsync(ctx.stage_in.ptr, in, in_len, hipMemcpyHostToDevice, ctx.stream));
  IlvEncResult r{};
  uint64_t needed = 0, n = in_len, src = reinterpret_cast<uint64_t>(ctx.stage_in.ptr);
  int64_t rc = ilv_encode_planes(ctx, &src, &n, 1, reinterpret_cast<uint64_t>(ctx.stage_out.ptr), bound, false, &r,
                                 &needed);
  if (rc < 0) return rc;
  if (r.len > out_len) return kBufferTooSmall;
  PTWM_HIP_TRY(hipMemcpyAsync(out, ctx.stage_out.ptr, r.len, hipMemcpyDeviceToHost, ctx.stream));
  PTWM_HIP_TRY(hipStreamSynchronize(ctx.stream));
  return (int64_t)r.len;
}

int64_t ptwm_plane_codec_v1_decode(const uint8_t* in, size_t in_len, uint8_t* out, size_t out_len) {
  if ((in_len && !in) || (out_len && !out)) return kInvalidInput;
  DeviceScope ds(kHostDevice);
  if (!ds.ok) return kMissingCapability;
  DevCtx& ctx = *ds.ctx;
  PTWM_HIP_TRY(ctx.stage_in.ensure(in_len + 16));
  PTWM_HIP_TRY(ctx.stage_out.ensure(out_len + 64));
  if (in_len) PTWM_HIP_TRY(hipMemcpyAsync(ctx.stage_in.ptr, in, in_len, hipMemcpyHostToDevice, ctx.stream));
  int64_t rc = ilv_decode_payload(ctx, reinterpret_cast<uint64_t>(ctx.stage_in.ptr), in_len,
                                  reinterpret_cast<uint64_t>(ctx.stage_out.ptr), out_len);
  if (rc <= 0) return rc;
  PTWM_HIP_TRY(hipMemcpyAsync(out, ctx.stage_out.ptr, (size_t)rc, hipMemcpyDeviceToHost, ctx.stream));
  PTWM_HIP_TRY(hipStreamSynchronize(ctx.stream));
  return rc;
}

int64_t ptwm_plane_codec_v1_decode_stateful(uint8_t state_format_version, const uint8_t* state_ptr,
                                            size_t state_len, const uint8_t* in, size_t in_len, uint8_t* out,
                                            size_t out_cap) {
  (void)state_format_version;
  (void)state_ptr;
  if (state_len != 0) return kInvalidInput;
  return ptwm_plane_codec_v1_decode(in, in_len, out, out_cap);
}

int64_t ptwm_mi355x_split_cuda(uint32_t chain, uint64_t in_dev_ptr, size_t in_len, const uint64_t* plane_dev_ptrs,
                               uint32_t n_planes, uint32_t device_ordinal) {
  int np = chain_planes(chain);
  if (np < 0 || (uint32_t)np != n_planes || !plane_dev_ptrs) return kInvalidInput;
  uint64_t ratio = (uint64_t)chain_ratio(chain);
  if (in_len % ratio) return kInvalidInput;
  uint64_t plane_len = in_len / ratio;
  if (plane_len == 0) return 0;
  DeviceScope ds(device_ordinal);
  if (!ds.ok) return kInvalidInput;
  uint8_t* pl[4] = {};
  for (int i = 0; i < np; ++i) pl[i] = reinterpret_cast<uint8_t*>(plane_dev_ptrs[i]);
  if (launch_split(chain, reinterpret_cast<const uint8_t*>(in_dev_ptr), plane_len, pl, ds.ctx->stream) !=
      hipSuccess)
    return kInvalidInput;
  PTWM_HIP_TRY(hipStreamSynchronize(ds.ctx->stream));
  return (int64_t)plane_len;
}

int64_t ptwm_mi355x_merge_cuda(uint32_t chain, const uint64_t* plane_dev_ptrs, uint32_t n_planes, size_t plane_len,
                               uint64_t out_dev_ptr, size_t out_cap, uint32_t device_ordinal) {
  int np = chain_planes(chain);
  if (np < 0 || (uint32_t)np != n_planes || !plane_dev_ptrs) return kInvalidInput;
  uint64_t out_len = (uint64_t)plane_len * (uint64_t)chain_ratio(chain);
  if (out_len > out_cap) return kBufferTooSmall;
  if (plane_len == 0) return 0;
  DeviceScope ds(device_ordinal);
  if (!ds.ok) return kInvalidInput;
  const uint8_t* pl[4] = {};
  for (int i = 0; i < np; ++i) pl[i] = reinterpret_cast<const uint8_t*>(plane_dev_ptrs[i]);
  DevCtx& ctx = *ds.ctx;
  if (ctx.profile) {
    PTWM_HIP_TRY(ctx.ensure_events());
    PTWM_HIP_TRY(hipEventRecord(ctx.ev[1], ctx.stream));
  }
  if (launch_merge(chain, pl, plane_len, reinterpret_cast<uint8_t*>(out_dev_ptr), ctx.stream) != hipSuccess)
    return kInvalidInput;
  if (ctx.profile) PTWM_HIP_TRY(hipEventRecord(ctx.ev[2], ctx.stream));
  PTWM_HIP_TRY(hipStreamSynchronize(ctx.stream));
  if (ctx.profile) {
    ctx.last_ms[0] = 0;
    PTWM_HIP_TRY(hipEventElapsedTime(&ctx.last_ms[1], ctx.ev[1], ctx.ev[2]));
    ctx.last_ms[2] = ctx.last_ms[1];
  }
  return (int64_t)out_len;
}

static int64_t encode_tensor_native(uint32_t family, uint32_t chain, uint64_t in_dev_ptr, size_t in_len,
                                    uint64_t out_dev_ptr, size_t out_cap, uint8_t* plan_out, size_t plan_cap,
                                    size_t* plan_len_out, uint64_t* needed_out, uint32_t device_ordinal) {
  const int np = chain_planes(chain);
  if (np < 0 || !plan_out || !plan_len_out) return kInvalidInput;
  const uint64_t ratio = (uint64_t)chain_ratio(chain);
  if (in_len % ratio || (in_dev_ptr & 15u) || (out_dev_ptr & 255u)) return kInvalidInput;
  const uint64_t plane_len = in_len / ratio;
  const size_t plan_len = 12 + 20 + (size_t)np * 32;
  if (plan_cap < plan_len) return kBufferTooSmall;
  DeviceScope ds(device_ordinal);
  if (!ds.ok) return kInvalidInput;
  DevCtx& ctx = *ds.ctx;
  // forward chain into plane scratch, then every plane through the encoder
  const uint64_t stride = (plane_len + 255) / 256 * 256;
  PTWM_HIP_TRY(ctx.enc_split.ensure(stride * np + 256));
  uint8_t* pl[4] = {};
  uint64_t srcs[4], lens[4];
  for (int i = 0; i < np; ++i) {
    pl[i] = static_cast<uint8_t*>(ctx.enc_split.ptr) + stride * i;
    srcs[i] = reinterpret_cast<uint64_t>(pl[i]);
    lens[i] = plane_len;
  }
  if (plane_len && launch_split(chain, reinterpret_cast<const uint8_t*>(in_dev_ptr), plane_len, pl, ctx.stream) !=
                       hipSuccess)
    return kInvalidInput;
  IlvEncResult r[4] = {};
  uint64_t needed = 0;
  int64_t rc = family == kFamilyHuff
                   ? ilv_encode_planes(ctx, srcs, lens, (uint32_t)np, out_dev_ptr, out_cap, true, r, &needed)
                   : rilv_encode_planes(ctx, srcs, lens, (uint32_t)np, out_dev_ptr, out_cap, true, r, &needed);
  if (rc == kBufferTooSmall && needed_out) *needed_out = needed;
  if (rc < 0) return rc;
  // decode plan (PTMD v1) for the one tensor
  uint8_t* o = plan_out;
  auto put = [&](const void* v, size_t k) {
    std::memcpy(o, v, k);
    o += k;
  };
  const uint32_t magic = 0x444D5450u, ntens = 1;
  const uint16_t ver = 1, flags = 0, tflags = 0;
  const uint64_t zero64 = 0, out_len = in_len;
  const uint8_t ch = (uint8_t)chain, npl = (uint8_t)np;
  put(&magic, 4); put(&ver, 2); put(&flags, 2); put(&ntens, 4);
  put(&zero64, 8); put(&out_len, 8); put(&ch, 1); put(&npl, 1); put(&tflags, 2);
  for (int i = 0; i < np; ++i) {
    const uint16_t codec = (uint16_t)r[i].codec, pf = 0;
    const uint32_t nch = 0;
    put(&codec, 2); put(&pf, 2); put(&nch, 4);
    put(&r[i].offset, 8); put(&r[i].len, 8); put(&plane_len, 8);
  }
  *plan_len_out = (size_t)(o - plan_out);
  return rc;
}

int64_t ptwm_mi355x_encode_tensor_cuda(uint32_t chain, uint64_t in_dev_ptr, size_t in_len, uint64_t out_dev_ptr,
                                       size_t out_cap, uint8_t* plan_out, size_t plan_cap, size_t* plan_len_out,
                                       uint64_t* needed_out, uint32_t device_ordinal) {
  return encode_tensor_native(kFamilyHuff, chain, in_dev_ptr, in_len, out_dev_ptr, out_cap, plan_out, plan_cap,
                              plan_len_out, needed_out, device_ordinal);
}

int64_t ptwm_mi355x_encode_tensor_rans_cuda(uint32_t chain, uint64_t in_dev_ptr, size_t in_len, uint64_t out_dev_ptr,
                                            size_t out_cap, uint8_t* plan_out, size_t plan_cap, size_t* plan_len_out,
                                            uint64_t* needed_out, uint32_t device_ordinal) {
  return encode_tensor_native(kFamilyRans, chain, in_dev_ptr, in_len, out_dev_ptr, out_cap, plan_out, plan_cap,
                              plan_len_out, needed_out, device_ordinal);
}

int64_t ptwm_mi355x_encode_tensors_cuda(uint32_t family, uint32_t n_tensors, const uint32_t* chains,
                                        const uint64_t* in_dev_ptrs, const uint64_t* in_lens, uint64_t out_dev_ptr,
                                        size_t out_cap, uint8_t* plan_out, size_t plan_cap, size_t* plan_len_out,
                                        uint64_t* needed_out, uint32_t device_ordinal) {
  if (family > kFamilyRans || !plan_out || !plan_len_out || (n_tensors && (!chains || !in_dev_ptrs || !in_lens)))
    return kInvalidInput;
  if (out_dev_ptr & 255u) return kInvalidInput;
  size_t plan_len = 12;
  for (uint32_t i = 0; i < n_tensors; ++i) {
    const int np = chain_planes(chains[i]);
    if (np < 0) return kInvalidInput;
    const uint64_t ratio = (uint64_t)chain_ratio(chains[i]);
    if (in_lens[i] % ratio || (in_dev_ptrs[i] & 15u)) return kInvalidInput;
    plan_len += 20 + (size_t)np * 32;
  }
  if (plan_cap < plan_len) return kBufferTooSmall;
  DeviceScope ds(device_ordinal);
  if (!ds.ok) return kInvalidInput;
  DevCtx& ctx = *ds.ctx;
  // Batches of tensors (at most kBatchBytes of input each, or one larger
  // tensor): forward chains of the batch into plane scratch, then every
  // plane of the batch through one encoder pass (one histogram, size and
  // encode launch each), payloads appended at 256-byte aligned offsets.
  const uint64_t kBatchBytes = ctx.enc_batch_bytes;
  std::vector<IlvEncResult> res;     // per plane, offsets relative to out_dev_ptr
  uint64_t out_used = 0, needed_total = 0;
  bool too_small = false;
  for (uint32_t b0 = 0; b0 < n_tensors;) {
    uint32_t b1 = b0;
    uint64_t scratch = 0;
    while (b1 < n_tensors && (b1 == b0 || scratch + in_lens[b1] + 1024 <= kBatchBytes)) {
      const uint64_t pl = in_lens[b1] / (uint64_t)chain_ratio(chains[b1]);
      scratch += (uint64_t)chain_planes(chains[b1]) * ((pl + 255) / 256 * 256);
      ++b1;
    }
    if (too_small) {
      // the output ran out in an earlier batch: only a size bound is
      // needed, and the stored size (n + 1) bounds every payload form
      for (uint32_t i = b0; i < b1; ++i) {
        const uint64_t pl = in_lens[i] / (uint64_t)chain_ratio(chains[i]);
        for (int k = 0; k < chain_planes(chains[i]); ++k) needed_total = (needed_total + 255) / 256 * 256 + pl + 1;
      }
      b0 = b1;
      continue;
    }
    PTWM_HIP_TRY(ctx.enc_split.ensure(scratch + 256));
    std::vector<uint64_t> srcs, lens;
    uint64_t so = 0;
    for (uint32_t i = b0; i < b1; ++i) {
      const int np = chain_planes(chains[i]);
      const uint64_t pl = in_lens[i] / (uint64_t)chain_ratio(chains[i]);
      uint8_t* p[4] = {};
      for (int k = 0; k < np; ++k) {
        p[k] = static_cast<uint8_t*>(ctx.enc_split.ptr) + so;
        srcs.push_back(reinterpret_cast<uint64_t>(p[k]));
        lens.push_back(pl);
        so += (pl + 255) / 256 * 256;
      }
      if (pl && launch_split(chains[i], reinterpret_cast<const uint8_t*>(in_dev_ptrs[i]), pl, p, ctx.stream) !=
                    hipSuccess)
        return kInvalidInput;
    }
    std::vector<IlvEncResult> r(srcs.size());
    uint64_t needed = 0;
    const uint64_t base = (out_used + 255) / 256 * 256;
    const uint64_t cap = out_cap > base ? out_cap - base : 0;
    int64_t rc = family == kFamilyHuff
                     ? ilv_encode_planes(ctx, srcs.data(), lens.data(), (uint32_t)srcs.size(), out_dev_ptr + base, cap,
                                         true, r.data(), &needed)
                     : rilv_encode_planes(ctx, srcs.data(), lens.data(), (uint32_t)srcs.size(), out_dev_ptr + base,
                                          cap, true, r.data(), &needed);
    if (rc == kBufferTooSmall) {
      // this batch's exact size (the encoder sized it); later batches are
      // only bounded (above)
      too_small = true;
      needed_total = base + needed;
    } else if (rc < 0) {
      return rc;
    } else {
      out_used = base + (uint64_t)rc;
      for (IlvEncResult& x : r) x.offset += base;
      res.insert(res.end(), r.begin(), r.end());
    }
    b0 = b1;
  }
  if (too_small) {
    if (needed_out) *needed_out = needed_total;
    return kBufferTooSmall;
  }
  // decode plan (PTMD v1): tensors restored back to back at 256-byte
  // aligned offsets, in the order given
  uint8_t* o = plan_out;
  auto put = [&](const void* v, size_t k) {
    std::memcpy(o, v, k);
    o += k;
  };
  const uint32_t magic = 0x444D5450u, ntens = n_tensors;
  const uint16_t ver = 1, flags = 0, tflags = 0;
  put(&magic, 4); put(&ver, 2); put(&flags, 2); put(&ntens, 4);
  uint64_t out_off = 0;
  size_t ri = 0;
  for (uint32_t i = 0; i < n_tensors; ++i) {
    const int np = chain_planes(chains[i]);
    const uint64_t pl = in_lens[i] / (uint64_t)chain_ratio(chains[i]);
    const uint64_t out_len = in_lens[i];
    const uint8_t ch = (uint8_t)chains[i], npl = (uint8_t)np;
    put(&out_off, 8); put(&out_len, 8); put(&ch, 1); put(&npl, 1); put(&tflags, 2);
    for (int k = 0; k < np; ++k, ++ri) {
      const uint16_t codec = (uint16_t)res[ri].codec, pf = 0;
      const uint32_t nch = 0;
      put(&codec, 2); put(&pf, 2); put(&nch, 4);
      put(&res[ri].offset, 8); put(&res[ri].len, 8); put(&pl, 8);
    }
    out_off = (out_off + out_len + 255) / 256 * 256;
  }
  *plan_len_out = (size_t)(o - plan_out);
  return (int64_t)out_used;
}

namespace {

// Plane op spec of the encoders: 0 none, else op | param << 8 (codes.h).
constexpr uint32_t op_of(uint32_t spec) { return spec & 0xFFu; }
constexpr uint32_t param_of(uint32_t spec) { return spec >> 8; }

bool op_spec_ok(uint32_t chain, uint32_t spec) {
  if (spec == 0) return true;
  const uint32_t op = op_of(spec), param = param_of(spec);
  if (chain != kChainIeee16Split2 && chain != kChainIeee32Split4 && chain != kChainPassthrough) return false;
  if (op == kPlaneOpPredictorXor) return param == 1 || param == 2;
  if (op == kPlaneOpIntDelta) return param == 1 || param == 2 || param == 4 || param == 8;
  return op == kPlaneOpMantissaZeroStrip && param >= 1 && param <= 7;
}

// PTMD plane flag bits of an op spec (plan_parse.cpp)
uint16_t op_flags(uint32_t spec) {
  if (spec == 0) return 0;
  const uint32_t op = op_of(spec), param = param_of(spec);
  const uint32_t code = op == kPlaneOpMantissaZeroStrip ? param : (uint32_t)__builtin_ctz(param);
  return (uint16_t)((op << 1) | (code << 3));
}

// Tensor-level encode into the reference's plane formats, plane p passed
// through the op ops[p] first.  With `trial`, ops is ignored and the
// reference's chain trial picks among the production split-chain variants
// (_chains.py:1146-1185; compressor.rs:504-640: every candidate forward and
// trial-encoded, the smallest total of plane payloads wins, the first on
// ties, a candidate whose forward fails is skipped); ops_out gets the
// chosen ops.
int64_t encode_tensor_ref(uint32_t chain, const uint16_t* plane_codecs, const uint16_t* ops_in, uint32_t n_planes,
                          bool trial, uint32_t chunk_size, uint64_t in_dev_ptr, size_t in_len, uint64_t out_dev_ptr,
                          size_t out_cap, uint8_t* plan_out, size_t plan_cap, size_t* plan_len_out,
                          uint64_t* needed_out, uint16_t* ops_out, uint32_t device_ordinal) {
  const int np = chain_planes(chain);
  if (np < 0 || !plan_out || !plan_len_out || !plane_codecs || n_planes != (uint32_t)np) return kInvalidInput;
  uint32_t codecs[4] = {0, 0, 0, 0};
  for (int p = 0; p < np; ++p) {
    codecs[p] = plane_codecs[p];
    if (codecs[p] != kCodecIdentity && codecs[p] != kCodecHuffman && codecs[p] != kCodecRans &&
        codecs[p] != PTWM_MI355X_CODEC_SELECT)
      return kUnsupported;
  }
  // the candidates: plane op specs per plane
  std::vector<std::array<uint32_t, 4>> cand;
  if (trial) {
    if (chain != kChainIeee16Split2 && chain != kChainIeee32Split4) return kUnsupported;
    const int ex = chain == kChainIeee16Split2 ? 1 : 3;  // the exponent plane (_chains.py:360-600)
    cand.push_back({0, 0, 0, 0});
    std::array<uint32_t, 4> c{0, 0, 0, 0};
    c[ex] = kPlaneOpIntDelta | 1u << 8;
    cand.push_back(c);
    c[ex] = kPlaneOpPredictorXor | 1u << 8;
    cand.push_back(c);
    for (uint32_t k = 1; k <= 4; ++k) cand.push_back({kPlaneOpMantissaZeroStrip | k << 8, 0, 0, 0});
  } else {
    std::array<uint32_t, 4> c{0, 0, 0, 0};
    for (int p = 0; p < np; ++p) {
      c[p] = ops_in ? ops_in[p] : 0u;
      if (!op_spec_ok(chain, c[p])) return kUnsupported;
    }
    cand.push_back(c);
  }
  const uint64_t ratio = (uint64_t)chain_ratio(chain);
  if (in_len % ratio || (in_dev_ptr & 15u) || (out_dev_ptr & 255u)) return kInvalidInput;
  const uint64_t plane_len = in_len / ratio;
  for (const auto& c : cand)
    for (int p = 0; p < np; ++p)
      if (c[p] && op_of(c[p]) != kPlaneOpMantissaZeroStrip && plane_len % param_of(c[p])) return kInvalidInput;
  // chunks: plane.chunks(chunk_size) (compressor.rs:316-381); 0 = unchunked
  const uint64_t cs = chunk_size ? chunk_size : (plane_len ? plane_len : 1);
  const uint64_t nch = chunk_size ? (plane_len == 0 ? 1 : (plane_len + cs - 1) / cs) : 1;
  if (nch > 0xFFFFFFFFull) return kInvalidInput;
  const size_t plan_len = 12 + 20 + (size_t)np * (32 + (chunk_size ? 8 * nch : 0));
  if (plan_cap < plan_len) {
    *plan_len_out = plan_len;
    return kBufferTooSmall;
  }
  DeviceScope ds(device_ordinal);
  if (!ds.ok) return kInvalidInput;
  DevCtx& ctx = *ds.ctx;
  // the distinct (plane, op) planes of every candidate: the split planes,
  // then one op output each
  struct Var {
    int plane;
    uint32_t spec;
    uint8_t* ptr;
    bool refused;
    uint64_t size;  // payload bytes of the plane with its codec (or the trial's choice)
    uint32_t codec;
  };
  std::vector<Var> vars;
  const auto var_of = [&](int p, uint32_t spec) {
    for (size_t i = 0; i < vars.size(); ++i)
      if (vars[i].plane == p && vars[i].spec == spec) return (int)i;
    vars.push_back(Var{p, spec, nullptr, false, 0, 0});
    return (int)vars.size() - 1;
  };
  for (int p = 0; p < np; ++p) var_of(p, 0);
  for (const auto& c : cand)
    for (int p = 0; p < np; ++p) var_of(p, c[p]);
  const uint64_t stride = (plane_len + 255) / 256 * 256;
  PTWM_HIP_TRY(ctx.enc_split.ensure(stride * vars.size() + 256));
  for (size_t i = 0; i < vars.size(); ++i) vars[i].ptr = static_cast<uint8_t*>(ctx.enc_split.ptr) + stride * i;
  uint8_t* pl[4] = {};
  for (int i = 0; i < np; ++i) pl[i] = vars[i].ptr;  // the first np vars are the split planes
  if (plane_len && launch_split(chain, reinterpret_cast<const uint8_t*>(in_dev_ptr), plane_len, pl, ctx.stream) !=
                       hipSuccess)
    return kInvalidInput;
  if (vars.size() > (size_t)np && plane_len) {
    std::vector<PlaneOpJob> jobs;
    for (size_t i = np; i < vars.size(); ++i)
      jobs.push_back(PlaneOpJob{reinterpret_cast<uint64_t>(pl[vars[i].plane]), reinterpret_cast<uint64_t>(vars[i].ptr),
                                plane_len, op_of(vars[i].spec), param_of(vars[i].spec), 0, 0});
    std::vector<uint32_t> refused;
    const int64_t rc = run_plane_ops(ctx, jobs, true, &refused);
    if (rc != kOk) return rc;
    for (size_t i = np; i < vars.size(); ++i) vars[i].refused = refused[i - np] != 0;
  }
  // sizes of every var the candidates need (trial) or the codecs' choice
  // (select.rs:27-64: Huffman, rANS and Identity in menu order, smallest
  // first wins)
  std::vector<int> chosen_var(np, -1);
  size_t best = 0;
  if (cand.size() == 1) {
    for (int p = 0; p < np; ++p) {
      chosen_var[p] = var_of(p, cand[0][p]);
      if (vars[chosen_var[p]].refused) return kInvalidInput;  // the forward op fails (mantissa_zero.rs)
    }
  }
  const bool need_sizes = cand.size() > 1;
  bool any_select = false;
  for (int p = 0; p < np; ++p) any_select |= codecs[p] == PTWM_MI355X_CODEC_SELECT;
  if (need_sizes || any_select) {
    std::vector<RefJob> tj;
    std::vector<std::pair<size_t, uint32_t>> tj_of;  // (var, codec)
    for (size_t i = 0; i < vars.size(); ++i) {
      const Var& V = vars[i];
      if (V.refused || plane_len == 0) continue;
      if (!need_sizes && chosen_var[V.plane] != (int)i) continue;
      const uint32_t c = codecs[V.plane];
      if (c == PTWM_MI355X_CODEC_SELECT || c == kCodecHuffman) {
        tj.push_back(RefJob{reinterpret_cast<uint64_t>(V.ptr), plane_len, kCodecHuffman});
        tj_of.emplace_back(i, kCodecHuffman);
      }
      if (c == PTWM_MI355X_CODEC_SELECT || c == kCodecRans) {
        tj.push_back(RefJob{reinterpret_cast<uint64_t>(V.ptr), plane_len, kCodecRans});
        tj_of.emplace_back(i, kCodecRans);
      }
    }
    std::vector<uint64_t> tl;
    if (!tj.empty()) {
      RefEncoder t;
      const int64_t rc = t.plan(ctx, tj, tl);
      if (rc < 0) return rc;
    }
    for (size_t i = 0; i < vars.size(); ++i) {
      Var& V = vars[i];
      const uint32_t c = codecs[V.plane];
      V.codec = c == PTWM_MI355X_CODEC_SELECT ? kCodecHuffman : c;
      V.size = plane_len;  // Identity (and an empty plane: 0 bytes against a 1-byte tag)
      if (plane_len == 0) {
        if (c == PTWM_MI355X_CODEC_SELECT) V.codec = kCodecIdentity;
        continue;
      }
      bool first = true;
      for (size_t k = 0; k < tj_of.size(); ++k) {
        if (tj_of[k].first != i) continue;
        if (first || tl[k] < V.size) {
          V.size = tl[k];
          V.codec = tj_of[k].second;
        }
        first = false;
      }
      if (c == PTWM_MI355X_CODEC_SELECT && plane_len < V.size) {
        V.size = plane_len;
        V.codec = kCodecIdentity;
      }
    }
    if (need_sizes) {
      // compressor.rs:589-593: the first candidate with the smallest total
      int bi = -1;
      for (size_t k = 0; k < cand.size(); ++k) {
        size_t total = 0;
        bool ok = true;
        for (int p = 0; p < np; ++p) {
          const Var& V = vars[var_of(p, cand[k][p])];
          ok &= !V.refused;
          total += V.size;
        }
        if (ok && (bi < 0 || total < best)) {
          bi = (int)k;
          best = total;
        }
      }
      if (bi < 0) return kInternal;  // the plain split never fails
      for (int p = 0; p < np; ++p) chosen_var[p] = var_of(p, cand[bi][p]);
    }
    for (int p = 0; p < np; ++p)
      if (codecs[p] == PTWM_MI355X_CODEC_SELECT) codecs[p] = vars[chosen_var[p]].codec;
  }
  uint32_t spec[4] = {0, 0, 0, 0};
  for (int p = 0; p < np; ++p) {
    pl[p] = vars[chosen_var[p]].ptr;
    spec[p] = vars[chosen_var[p]].spec;
    if (ops_out) ops_out[p] = (uint16_t)spec[p];
  }
  // one job per coded chunk; Identity payloads are the bytes themselves
  std::vector<RefJob> jobs;
  std::vector<int> job_of(np * nch, -1);
  for (int p = 0; p < np; ++p)
    for (uint64_t k = 0; k < nch; ++k) {
      const uint64_t a = k * cs, b = std::min(plane_len, a + cs);
      if (codecs[p] == kCodecIdentity) continue;
      job_of[p * nch + k] = (int)jobs.size();
      jobs.push_back(RefJob{reinterpret_cast<uint64_t>(pl[p]) + a, b - a, codecs[p]});
    }
  RefEncoder enc;
  std::vector<uint64_t> plen;
  int64_t rc = enc.plan(ctx, jobs, plen);
  if (rc < 0) return rc;
  // layout: planes at 256-byte boundaries; a chunked plane is its frames
  // [ver u8 = 0][state_len u32 = 0][payload] back to back
  std::vector<uint64_t> dst(jobs.size(), 0), poff(np), plen_total(np);
  std::vector<std::vector<std::pair<uint32_t, uint32_t>>> table(np);
  std::vector<std::pair<uint64_t, std::vector<uint8_t>>> literal;
  std::vector<RefCopyOp> copies;
  uint64_t off = 0;
  for (int p = 0; p < np; ++p) {
    off = (off + 255) / 256 * 256;
    poff[p] = off;
    uint64_t q = 0;
    for (uint64_t k = 0; k < nch; ++k) {
      const uint64_t a = k * cs, b = std::min(plane_len, a + cs);
      if (chunk_size) {
        if (q > 0xFFFFFFFFull) return kInvalidInput;
        table[p].emplace_back((uint32_t)q, (uint32_t)(b - a));
        literal.emplace_back(out_dev_ptr + off + q, std::vector<uint8_t>(5, 0));
        q += 5;
      }
      const int j = job_of[p * nch + k];
      if (j >= 0) {
        dst[j] = out_dev_ptr + off + q;
        q += plen[j];
      } else {
        copies.push_back(RefCopyOp{reinterpret_cast<uint64_t>(pl[p]) + a, out_dev_ptr + off + q, b - a, ~0ull});
        q += b - a;
      }
    }
    plen_total[p] = q;
    off += q;
  }
  if (off > out_cap) {
    if (needed_out) *needed_out = off;
    return kBufferTooSmall;
  }
  rc = enc.write(ctx, dst, literal, copies);
  if (rc < 0) return rc;
  uint8_t* o = plan_out;
  auto put = [&](const void* v, size_t k) {
    std::memcpy(o, v, k);
    o += k;
  };
  const uint32_t magic = 0x444D5450u, ntens = 1;
  const uint16_t ver = 1, flags = 0, tflags = 0;
  const uint64_t zero64 = 0, out_len = in_len;
  const uint8_t ch = (uint8_t)chain, npl = (uint8_t)np;
  put(&magic, 4); put(&ver, 2); put(&flags, 2); put(&ntens, 4);
  put(&zero64, 8); put(&out_len, 8); put(&ch, 1); put(&npl, 1); put(&tflags, 2);
  for (int p = 0; p < np; ++p) {
    const uint16_t codec = (uint16_t)codecs[p], pf = (uint16_t)((chunk_size ? 1 : 0) | op_flags(spec[p]));
    const uint32_t n_ch = chunk_size ? (uint32_t)nch : 0;
    put(&codec, 2); put(&pf, 2); put(&n_ch, 4);
    put(&poff[p], 8); put(&plen_total[p], 8); put(&plane_len, 8);
    for (const auto& e : table[p]) {
      put(&e.first, 4);
      put(&e.second, 4);
    }
  }
  *plan_len_out = (size_t)(o - plan_out);
  return (int64_t)off;
}

}  // namespace

int64_t ptwm_mi355x_encode_tensor_ref_cuda(uint32_t chain, const uint16_t* plane_codecs, uint32_t n_codecs,
                                           uint32_t chunk_size, uint64_t in_dev_ptr, size_t in_len,
                                           uint64_t out_dev_ptr, size_t out_cap, uint8_t* plan_out, size_t plan_cap,
                                           size_t* plan_len_out, uint64_t* needed_out, uint32_t device_ordinal) {
  return encode_tensor_ref(chain, plane_codecs, nullptr, n_codecs, false, chunk_size, in_dev_ptr, in_len, out_dev_ptr,
                           out_cap, plan_out, plan_cap, plan_len_out, needed_out, nullptr, device_ordinal);
}

int64_t ptwm_mi355x_encode_tensor_ref_ops_cuda(uint32_t chain, const uint16_t* plane_codecs, const uint16_t* plane_ops,
                                               uint32_t n_planes, uint32_t chain_trial, uint32_t chunk_size,
                                               uint64_t in_dev_ptr, size_t in_len, uint64_t out_dev_ptr,
                                               size_t out_cap, uint8_t* plan_out, size_t plan_cap,
                                               size_t* plan_len_out, uint64_t* needed_out, uint16_t* ops_out,
                                               uint32_t device_ordinal) {
  if (chain_trial > 1 || (!chain_trial && !plane_ops)) return kInvalidInput;
  return encode_tensor_ref(chain, plane_codecs, plane_ops, n_planes, chain_trial != 0, chunk_size, in_dev_ptr, in_len,
                           out_dev_ptr, out_cap, plan_out, plan_cap, plan_len_out, needed_out, ops_out,
                           device_ordinal);
}

int64_t ptwm_mi355x_plane_crc32_cuda(uint32_t chain, uint64_t in_dev_ptr, size_t in_len, uint32_t* crc_out,
                                     uint32_t n_out, uint32_t device_ordinal) {
  const int np = chain_planes(chain);
  if (np < 0 || !crc_out || n_out < (uint32_t)np) return kInvalidInput;
  const uint64_t ratio = (uint64_t)chain_ratio(chain);
  if (in_len % ratio || (in_len && !in_dev_ptr)) return kInvalidInput;
  const uint64_t n = in_len / ratio;
  DeviceScope ds(device_ordinal);
  if (!ds.ok) return kInvalidInput;
  DevCtx& ctx = *ds.ctx;
  uint64_t src = in_dev_ptr;
  if (n && (src & 15u)) {  // the kernels read dwordx4: realign into staging
    PTWM_HIP_TRY(ctx.stage_in.ensure(in_len + 16));
    PTWM_HIP_TRY(hipMemcpyAsync(ctx.stage_in.ptr, reinterpret_cast<const void*>(src), in_len,
                                hipMemcpyDeviceToDevice, ctx.stream));
    src = reinterpret_cast<uint64_t>(ctx.stage_in.ptr);
  }
  std::vector<CrcTask> tasks;
  if (crc_chain_supported(chain)) {
    tasks.push_back(CrcTask{src, n, chain});
  } else {  // nibble chains: forward chain into plane scratch, then each plane
    const uint64_t stride = (n + 255) / 256 * 256;
    PTWM_HIP_TRY(ctx.enc_split.ensure(stride * np + 256));
    uint8_t* pl[4] = {};
    for (int i = 0; i < np; ++i) {
      pl[i] = static_cast<uint8_t*>(ctx.enc_split.ptr) + stride * i;
      tasks.push_back(CrcTask{reinterpret_cast<uint64_t>(pl[i]), n, kChainPassthrough});
    }
    if (n && launch_split(chain, reinterpret_cast<const uint8_t*>(src), n, pl, ctx.stream) != hipSuccess)
      return kInvalidInput;
  }
  std::vector<uint32_t> crcs;
  const int64_t rc = crc32_planes(ctx, tasks, crcs);
  if (rc != kOk) return rc;
  if (crcs.size() != (size_t)np) return kInternal;
  for (int i = 0; i < np; ++i) crc_out[i] = crcs[i];
  return np;
}

int64_t ptwm_mi355x_xxh64_cuda(uint64_t in_dev_ptr, size_t in_len, uint64_t* hash_out, uint32_t device_ordinal) {
  if (!hash_out || (in_len && !in_dev_ptr)) return kInvalidInput;
  DeviceScope ds(device_ordinal);
  if (!ds.ok) return kInvalidInput;
  std::vector<uint64_t> h;
  const int64_t rc = xxh64_buffers(*ds.ctx, {HashTask{in_dev_ptr, in_len}}, h);
  if (rc != kOk) return rc;
  *hash_out = h[0];
  return 0;
}

int64_t ptwm_mi355x_set_encode_batch_bytes(uint64_t bytes, uint32_t device_ordinal) {
  DeviceScope ds(device_ordinal);
  if (!ds.ok) return kInvalidInput;
  ds.ctx->enc_batch_bytes = bytes ? bytes : kDefaultEncBatchBytes;
  return 0;
}

int64_t ptwm_mi355x_use_stream(uint64_t stream, uint32_t use, uint32_t device_ordinal) {
  if (!get_ctx(device_ordinal)) return kInvalidInput;
  t_stream.dev = device_ordinal;
  t_stream.stream = stream;
  t_stream.set = use != 0;
  return 0;
}

int64_t ptwm_mi355x_stream_wait(uint64_t producer_stream, uint32_t device_ordinal) {
  DeviceScope ds(device_ordinal);
  if (!ds.ok) return kInvalidInput;
  DevCtx& ctx = *ds.ctx;
  hipStream_t prod = reinterpret_cast<hipStream_t>(producer_stream);
  if (prod == ctx.stream) return 0;
  if (!ctx.order_ev) note_alloc();
  if (!ctx.order_ev) PTWM_HIP_TRY(hipEventCreateWithFlags(&ctx.order_ev, hipEventDisableTiming));
  PTWM_HIP_TRY(hipEventRecord(ctx.order_ev, prod));
  PTWM_HIP_TRY(hipStreamWaitEvent(ctx.stream, ctx.order_ev, 0));
  return 0;
}

int64_t ptwm_mi355x_device_init(uint32_t device_ordinal) {
  DevCtx* c = get_ctx(device_ordinal);
  if (!c) return kInvalidInput;
  return c->noalloc_dev && c->noalloc_status ? 0 : kMissingCapability;
}

uint64_t ptwm_mi355x_alloc_calls(void) { return alloc_calls(); }

int64_t ptwm_mi355x_decode_stats(uint32_t device_ordinal, uint64_t* out, size_t n) {
  if (n && !out) return kInvalidInput;
  DeviceScope ds(device_ordinal);
  if (!ds.ok) return kInvalidInput;
  const uint64_t v[3] = {ds.ctx->sync_accepted, ds.ctx->sync_fallbacks, ds.ctx->sync_extra_rounds};
  for (size_t i = 0; i < n && i < 3; ++i) out[i] = v[i];
  return 3;
}

int64_t ptwm_mi355x_set_profiling(uint32_t device_ordinal, uint32_t on) {
  DeviceScope ds(device_ordinal);
  if (!ds.ok) return kInvalidInput;
  ds.ctx->profile = on != 0;
  return 0;
}

int64_t ptwm_mi355x_last_kernel_ms(uint32_t device_ordinal, float* out3) {
  if (!out3) return kInvalidInput;
  DeviceScope ds(device_ordinal);
  if (!ds.ok) return kInvalidInput;
  for (int i = 0; i < 3; ++i) out3[i] = ds.ctx->last_ms[i];
  return 0;
}

}  // extern "C"
