// runtime.hip -- device contexts, scratch memory, decode-plan parsing and
// execution for the reference plane formats.
//
// A decode plan describes one or more tensors as the container stores them
// (container.rs:1795-2196): per tensor its chain (which fixes the inverse
// merge) and per plane its codec id, payload location, decoded length and,
// for chunked planes, the chunk table (plane_record.rs:16-20).  Every
// independently coded unit becomes one DecodeJob; all jobs of all tensors go
// to the device in one launch, then each tensor is merged.
#include <hip/hip_runtime.h>

#include <array>
#include <atomic>
#include <cstring>
#include <memory>

#include "decode_sync.h"
#include "ilv_host.h"
#include "integrity.h"
#include "plane_ops.h"
#include "runtime.h"

namespace ptwm {

namespace {
std::atomic<uint64_t> g_alloc_calls{0};
}
void note_alloc() { g_alloc_calls.fetch_add(1, std::memory_order_relaxed); }
uint64_t alloc_calls() { return g_alloc_calls.load(std::memory_order_relaxed); }

hipError_t DeviceBuffer::ensure(size_t bytes) {
  if (bytes <= cap && ptr) return hipSuccess;
  if (borrowed) return hipErrorOutOfMemory;
  if (ptr) {
    (void)hipFree(ptr);
    ptr = nullptr;
    cap = 0;
  }
  size_t want = bytes < 4096 ? 4096 : bytes;
  note_alloc();
  hipError_t e = hipMalloc(&ptr, want);
  if (e == hipSuccess) cap = want;
  return e;
}
DeviceBuffer::~DeviceBuffer() {}

hipError_t PinnedBuffer::ensure(size_t bytes) {
  if (bytes <= cap && ptr) return hipSuccess;
  if (borrowed) return hipErrorOutOfMemory;
  if (ptr) {
    (void)hipHostFree(ptr);
    ptr = nullptr;
    cap = 0;
  }
  size_t want = bytes < 4096 ? 4096 : bytes;
  note_alloc();
  hipError_t e = hipHostMalloc(&ptr, want, flags);
  if (e == hipSuccess) cap = want;
  return e;
}
PinnedBuffer::~PinnedBuffer() {}

hipError_t DevCtx::ensure_events() {
  for (auto& e : ev)
    if (!e) {
      note_alloc();
      hipError_t r = hipEventCreate(&e);
      if (r != hipSuccess) return r;
    }
  return hipSuccess;
}

hipError_t DevCtx::ensure_side() {
  if (!side_stream) {
    note_alloc();
    // default priority: mixing stream priorities is avoided on purpose
    hipError_t e = hipStreamCreateWithFlags(&side_stream, hipStreamNonBlocking);
    if (e != hipSuccess) return e;
  }
  for (hipEvent_t* ev : {&side_fork, &side_join})
    if (!*ev) {
      note_alloc();
      hipError_t e = hipEventCreateWithFlags(ev, hipEventDisableTiming);
      if (e != hipSuccess) return e;
    }
  return hipSuccess;
}

namespace {
std::mutex g_ctx_mu;
std::array<std::unique_ptr<DevCtx>, 64> g_ctx;

// Device scratch of the allocation-free decode: one copy per device (the
// code object's data segment), held until the process ends.  Host code
// never passes this name to a kernel or copy: get_ctx resolves each
// device's copy to its device address once (DevCtx::noalloc_dev), and only
// that address is used.
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
}  // namespace

DevCtx* find_ctx(uint32_t ord) {
  if (ord >= g_ctx.size()) return nullptr;
  std::lock_guard<std::mutex> lk(g_ctx_mu);
  return g_ctx[ord].get();
}

DevCtx* get_ctx(uint32_t ord) {
  if (ord >= g_ctx.size()) return nullptr;
  std::lock_guard<std::mutex> lk(g_ctx_mu);
  if (g_ctx[ord]) return g_ctx[ord].get();
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || (int)ord >= n) return nullptr;
  int prev = 0;
  (void)hipGetDevice(&prev);
  if (hipSetDevice((int)ord) != hipSuccess) return nullptr;
  auto ctx = std::make_unique<DevCtx>();
  ctx->dev = (int)ord;
  // default priority: mixing stream priorities is avoided on purpose
  note_alloc();
  if (hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking) != hipSuccess) {
    (void)hipSetDevice(prev);
    return nullptr;
  }
  ctx->stream = ctx->own_stream;
  ctx->h_ilv_status.flags = hipHostMallocCoherent;
  ctx->h_job_status.flags = hipHostMallocCoherent;
  // the allocation-free decode's scratch on this device (the device is
  // current): its address, or null, and the entry point then reports
  // MissingCapability
  void* sp = nullptr;
  note_alloc();
  if (hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch)) == hipSuccess && sp &&
      hipHostMalloc(&ctx->noalloc_status, kNoAllocStatusBytes, hipHostMallocCoherent) == hipSuccess) {
    ctx->noalloc_dev = static_cast<uint8_t*>(sp);
    ctx->noalloc_host.reset(new uint8_t[kNoAllocHostBytes]);
  } else {
    (void)hipGetLastError();
  }
  (void)hipSetDevice(prev);
  g_ctx[ord] = std::move(ctx);
  return g_ctx[ord].get();
}


static inline uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

bool fused_eligible(const PlanTensor& T, uint64_t out_dev) {
  bool any_huff = false, any_rans = false, ok = ((out_dev + T.out_offset) & 15u) == 0;
  for (const PlanPlane& P : T.planes) {
    if (P.chunked || P.op != kPlaneOpNone) ok = false;
    if (P.codec == kCodecHuffIlv) any_huff = true;
    else if (P.codec == kCodecRansIlv) any_rans = true;
    else if (P.codec != kCodecIdentity || P.payload_len != P.plane_len) ok = false;
  }
  // one codec family per fused tensor; a plane CRC is checked on the
  // restored tensor where the chain is a bijection on plane bytes (other
  // chains keep their planes in scratch)
  return ok && any_huff != any_rans && (!T.has_crc || crc_chain_supported(T.chain));
}

namespace {

// Views of the fixed scratch in place of the device context's grow-only
// buffers for the length of one allocation-free call; the context's own
// buffers come back when it ends.
struct Borrow {
  DeviceBuffer* dst[9];
  DeviceBuffer saved[9];
  PinnedBuffer* hdst[4];
  PinnedBuffer hsaved[4];
  bool tab_ready;
  DevCtx& ctx;
  explicit Borrow(DevCtx& c) : ctx(c) {
    uint8_t* d = c.noalloc_dev;
    struct View {
      DeviceBuffer* b;
      uint64_t off, len;
    } v[9] = {{&c.crc_tab, kNoAllocTabOff, kNoAllocTabBytes},
              {&c.ilv_args, kNoAllocArgsOff, kNoAllocArgsBytes},
              {&c.crc_args, kNoAllocCrcArgsOff, kNoAllocCrcArgsBytes},
              {&c.crc_comb, kNoAllocCombOff, kNoAllocCombBytes},
              {&c.planes, kNoAllocStubOff, 1024},
              {&c.jobs, kNoAllocStubOff + 1024, 1024},
              {&c.status, kNoAllocStubOff + 2048, 1024},
              {&c.crc_part, kNoAllocPartOff, kNoAllocPartBytes},
              {&c.ilv_realign, 0, 0}};
    for (int i = 0; i < 9; ++i) {
      dst[i] = v[i].b;
      saved[i] = *v[i].b;
      v[i].b->ptr = v[i].len ? d + v[i].off : nullptr;
      v[i].b->cap = v[i].len;
      v[i].b->borrowed = true;
    }
    uint8_t* h = c.noalloc_host.get();
    PinnedBuffer* hb[4] = {&c.h_ilv, &c.h_jobs, &c.h_status, &c.h_ilv_status};
    uint8_t* const hbase[4] = {h, h, h, static_cast<uint8_t*>(c.noalloc_status)};
    const uint64_t hoff[4] = {0, kNoAllocHostBytes - 2048, kNoAllocHostBytes - 1024, 0};
    const uint64_t hlen[4] = {kNoAllocHostBytes - 2048, 1024, 1024, kNoAllocStatusBytes};
    for (int i = 0; i < 4; ++i) {
      hdst[i] = hb[i];
      hsaved[i] = *hb[i];
      hb[i]->ptr = hbase[i] + hoff[i];
      hb[i]->cap = hlen[i];
      hb[i]->borrowed = true;
    }
    tab_ready = c.crc_tab_ready;
    c.crc_tab_ready = c.noalloc_tab_ready;
  }
  ~Borrow() {
    ctx.noalloc_tab_ready = ctx.crc_tab_ready;
    ctx.crc_tab_ready = tab_ready;
    for (int i = 0; i < 9; ++i) *dst[i] = saved[i];
    for (int i = 0; i < 4; ++i) *hdst[i] = hsaved[i];
  }
};

}  // namespace

int64_t execute_plan_noalloc(DevCtx& ctx, const Plan& plan, uint64_t in_dev, uint64_t out_dev) {
  if (!ctx.noalloc_dev || !ctx.noalloc_host) return kMissingCapability;
  if (plan.tensors.size() > kNoAllocMaxTensors) return kUnsupported;
  uint64_t crc_blocks = 0;
  for (const PlanTensor& T : plan.tensors) {
    if (T.has_hash || !fused_eligible(T, out_dev)) return kUnsupported;
    bool rans = false;
    for (const PlanPlane& P : T.planes) {
      rans |= P.codec == kCodecRansIlv;
      if (P.codec != kCodecIdentity && ((in_dev + P.payload_offset) & 3u)) return kUnsupported;
    }
    if (T.has_crc && !rans) crc_blocks += (T.planes[0].plane_len + kIlvBlock - 1) / kIlvBlock;
  }
  if (crc_blocks > kNoAllocMaxCrcBlocks) return kUnsupported;
  Borrow b(ctx);
  return execute_plan(ctx, plan, in_dev, out_dev);
}

namespace {

// The five header bytes [ver u8][state_len u32] of each chunk frame.
__global__ void gather_chunk_heads(const uint64_t* __restrict__ addr, uint32_t n, uint8_t* __restrict__ out) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint64_t a = addr[i];
#pragma unroll
  for (uint32_t k = 0; k < 5; ++k) out[8ull * i + k] = g_ld<uint8_t>(a + k);
}

// Payload ranges of the chunk frames of GPU-native planes (compressor.rs:
// 316-381 frames [ver][state_len u32][state][payload]; container.rs:
// 1975-2050 reads them), for the tensors that hold such planes.  The
// headers live in device memory: one gather kernel and one copy bring them
// over.  A native chunk carries no codec state (the codecs are stateless,
// as the plane codec entry points require); an Identity chunk with state
// keeps its frame for the exact path.  Per tensor, per plane, per chunk:
// the payload's device address and length (len = UINT64_MAX: keep framed).
struct ChunkRanges {
  std::vector<std::vector<std::vector<std::pair<uint64_t, uint64_t>>>> r;  // [t][p][k]
};

bool native_codec(uint32_t c) { return c == kCodecHuffIlv || c == kCodecRansIlv; }

int64_t chunk_ranges(DevCtx& ctx, const Plan& plan, uint64_t in_dev, ChunkRanges& cr) {
  const size_t nt = plan.tensors.size();
  cr.r.assign(nt, {});
  std::vector<uint64_t> addr;
  for (size_t t = 0; t < nt; ++t) {
    const PlanTensor& T = plan.tensors[t];
    bool any = false;
    for (const PlanPlane& P : T.planes) any |= P.chunked && native_codec(P.codec);
    if (!any) continue;
    cr.r[t].resize(T.planes.size());
    for (size_t p = 0; p < T.planes.size(); ++p) {
      const PlanPlane& P = T.planes[p];
      if (!P.chunked || !(native_codec(P.codec) || P.codec == kCodecIdentity)) continue;
      for (size_t k = 0; k < P.chunks.size(); ++k) {
        const uint64_t a = P.chunks[k].offset_in_payload;
        const uint64_t b = k + 1 < P.chunks.size() ? P.chunks[k + 1].offset_in_payload : P.payload_len;
        if (b - a < 5) return kInvalidInput;  // container.rs:2011-2015
        addr.push_back(in_dev + P.payload_offset + a);
      }
    }
  }
  if (addr.empty()) return kOk;
  const uint32_t n = (uint32_t)addr.size();
  PTWM_HIP_TRY(ctx.chunk_addr.ensure(8ull * n));
  PTWM_HIP_TRY(ctx.chunk_head.ensure(8ull * n));
  PTWM_HIP_TRY(ctx.h_chunk.ensure(8ull * n));
  hipStream_t s = ctx.stream;
  std::memcpy(ctx.h_chunk.ptr, addr.data(), 8ull * n);
  PTWM_HIP_TRY(hipMemcpyAsync(ctx.chunk_addr.ptr, ctx.h_chunk.ptr, 8ull * n, hipMemcpyHostToDevice, s));
  hipLaunchKernelGGL(gather_chunk_heads, dim3((n + 255) / 256), dim3(256), 0, s,
                     static_cast<const uint64_t*>(ctx.chunk_addr.ptr), n, static_cast<uint8_t*>(ctx.chunk_head.ptr));
  PTWM_HIP_TRY(hipGetLastError());
  PTWM_HIP_TRY(hipMemcpyAsync(ctx.h_chunk.ptr, ctx.chunk_head.ptr, 8ull * n, hipMemcpyDeviceToHost, s));
  PTWM_HIP_TRY(hipStreamSynchronize(s));
  const uint8_t* h = static_cast<const uint8_t*>(ctx.h_chunk.ptr);
  size_t j = 0;
  for (size_t t = 0; t < nt; ++t) {
    if (cr.r[t].empty()) continue;
    const PlanTensor& T = plan.tensors[t];
    for (size_t p = 0; p < T.planes.size(); ++p) {
      const PlanPlane& P = T.planes[p];
      if (!P.chunked || !(native_codec(P.codec) || P.codec == kCodecIdentity)) continue;
      auto& v = cr.r[t][p];
      for (size_t k = 0; k < P.chunks.size(); ++k, ++j) {
        const uint64_t a = P.chunks[k].offset_in_payload;
        const uint64_t b = k + 1 < P.chunks.size() ? P.chunks[k + 1].offset_in_payload : P.payload_len;
        const uint8_t* hd = h + 8 * j;
        const uint64_t sl = (uint64_t)hd[1] | ((uint64_t)hd[2] << 8) | ((uint64_t)hd[3] << 16) | ((uint64_t)hd[4] << 24);
        if (b - a - 5 < sl) return kInvalidInput;  // state_len past the frame (container.rs:2019-2023)
        if (sl != 0) {
          if (native_codec(P.codec)) return kInvalidInput;  // a stateless codec given state
          v.emplace_back(0, UINT64_MAX);
          continue;
        }
        v.emplace_back(in_dev + P.payload_offset + a + 5, b - a - 5);
      }
    }
  }
  return kOk;
}

// A tensor whose planes are all chunked GPU-native / Identity planes of one
// family with the same chunk boundaries, every chunk but the last a whole
// number of 16384-symbol blocks, decodes in the fused route as one
// sub-tensor per chunk: chunk k of every plane restores elements
// [a_k, a_k + size_k) straight into the output, and the CRC block partials
// of the sub-tensors follow each other as those of the whole tensor would.
bool chunked_fused_eligible(const PlanTensor& T, uint64_t out_dev, const ChunkRanges& cr, size_t t) {
  if (cr.r[t].empty() || ((out_dev + T.out_offset) & 15u)) return false;
  bool any_huff = false, any_rans = false;
  const PlanPlane& P0 = T.planes[0];
  for (size_t p = 0; p < T.planes.size(); ++p) {
    const PlanPlane& P = T.planes[p];
    if (!P.chunked || P.chunks.size() != P0.chunks.size() || P.op != kPlaneOpNone) return false;
    if (P.codec == kCodecHuffIlv) any_huff = true;
    else if (P.codec == kCodecRansIlv) any_rans = true;
    else if (P.codec != kCodecIdentity) return false;
    for (size_t k = 0; k < P.chunks.size(); ++k) {
      if (P.chunks[k].decoded_size != P0.chunks[k].decoded_size) return false;
      if (k + 1 < P.chunks.size() && P.chunks[k].decoded_size % kIlvBlock) return false;
      const auto& rg = cr.r[t][p][k];
      if (rg.second == UINT64_MAX) return false;
      if (P.codec == kCodecIdentity && rg.second != P.chunks[k].decoded_size) return false;
    }
  }
  return any_huff != any_rans && (!T.has_crc || crc_chain_supported(T.chain));
}

}  // namespace

int64_t execute_plan(DevCtx& ctx, const Plan& plan, uint64_t in_dev, uint64_t out_dev) {
  // Route 1 (fused): a tensor whose planes are all unchunked Identity or
  // GPU-native payloads of one codec family (huff_ilv or rans_ilv), with at
  // least one coded plane, is decoded and merged in one pass by that
  // family's kernel.
  // Route 2 (exact): every other tensor; reference-format planes become
  // DecodeJobs into plane scratch (GPU-native planes decode into scratch
  // through their fused kernel's passthrough chain), then the merge kernel
  // runs.
  const size_t nt = plan.tensors.size();
  for (const PlanTensor& T : plan.tensors)
    for (const PlanPlane& P : T.planes) {
      if (!plane_op_supported(P.op, P.op_param)) return kUnsupported;
      // an Order1ScaleAC state is at most 32 + 512 * 257 bytes
      // (order1_scale_ac.rs:159-182): a longer one is malformed
      if (P.has_state && P.state_len > 32u + 512u * 257u) return kInvalidInput;
    }
  std::vector<IlvTensor> ilv;
  std::vector<char> fused(nt, 0);
  // huff_ilv tensors with plane CRCs: the decode kernel also writes the CRC
  // partials of their whole blocks (tensor t's from block crc_first[t])
  std::vector<uint32_t> crc_first(nt, kIlvNoCrc);
  uint64_t crc_blocks = 0;
  ChunkRanges cr;
  {
    const int64_t rc = chunk_ranges(ctx, plan, in_dev, cr);
    if (rc != kOk) return rc;
  }
  for (size_t t = 0; t < nt; ++t) {
    const PlanTensor& T = plan.tensors[t];
    if (!fused_eligible(T, out_dev)) {
      if (!chunked_fused_eligible(T, out_dev, cr, t)) continue;
      // one sub-tensor per chunk (chunked_fused_eligible)
      bool any_rans = false;
      for (const PlanPlane& P : T.planes) any_rans |= P.codec == kCodecRansIlv;
      fused[t] = 1;
      const uint64_t n = T.planes[0].plane_len;
      if (T.has_crc && !any_rans && n > 0) {
        crc_first[t] = (uint32_t)crc_blocks;
        crc_blocks += (n + kIlvBlock - 1) / kIlvBlock;
        if (crc_blocks > 0xFFFFFFFEull) return kInvalidInput;
      }
      const uint32_t coded_codec = any_rans ? kCodecRansIlv : kCodecHuffIlv;
      const uint64_t ratio = (uint64_t)chain_ratio(T.chain);
      uint64_t a = 0;
      for (size_t k = 0; k < T.planes[0].chunks.size(); ++k) {
        IlvTensor X{};
        X.out = out_dev + T.out_offset + a * ratio;
        X.n = T.planes[0].chunks[k].decoded_size;
        X.chain = T.chain;
        X.n_planes = (uint32_t)T.planes.size();
        X.family = any_rans ? kFamilyRans : kFamilyHuff;
        X.crc_first = crc_first[t] == kIlvNoCrc ? kIlvNoCrc : crc_first[t] + (uint32_t)(a / kIlvBlock);
        for (size_t p = 0; p < T.planes.size(); ++p) {
          X.planes[p].base = cr.r[t][p][k].first;
          X.planes[p].len = cr.r[t][p][k].second;
          X.planes[p].coded = T.planes[p].codec == coded_codec ? 1 : 0;
          X.planes[p].lut = (uint32_t)p;
        }
        if (X.n > 0) ilv.push_back(X);
        a += X.n;
      }
      continue;
    }
    bool any_rans = false;
    for (const PlanPlane& P : T.planes) any_rans |= P.codec == kCodecRansIlv;
    fused[t] = 1;
    IlvTensor X{};
    X.out = out_dev + T.out_offset;
    X.n = T.planes[0].plane_len;
    X.chain = T.chain;
    X.n_planes = (uint32_t)T.planes.size();
    X.family = any_rans ? kFamilyRans : kFamilyHuff;
    X.crc_first = kIlvNoCrc;
    if (T.has_crc && !any_rans && X.n > 0) {
      X.crc_first = crc_first[t] = (uint32_t)crc_blocks;
      crc_blocks += (X.n + kIlvBlock - 1) / kIlvBlock;
      if (crc_blocks > 0xFFFFFFFEull) return kInvalidInput;
    }
    const uint32_t coded_codec = any_rans ? kCodecRansIlv : kCodecHuffIlv;
    for (size_t p = 0; p < T.planes.size(); ++p) {
      X.planes[p].base = in_dev + T.planes[p].payload_offset;
      X.planes[p].len = T.planes[p].payload_len;
      X.planes[p].coded = T.planes[p].codec == coded_codec ? 1 : 0;
      X.planes[p].lut = (uint32_t)p;
    }
    ilv.push_back(X);
  }
  // Pass 1 (exact route): lay out plane scratch and count jobs.  A plane
  // needs scratch unless it is a single unchunked Identity payload whose
  // (16-byte aligned) bytes can feed the merge directly from the input.
  constexpr uint64_t kDirect = UINT64_MAX;
  std::vector<std::vector<uint64_t>> scratch_off(nt);
  uint64_t scratch_bytes = 0;
  size_t n_jobs = 0;
  for (size_t t = 0; t < nt; ++t) {
    if (fused[t]) continue;
    const PlanTensor& T = plan.tensors[t];
    scratch_off[t].assign(T.planes.size(), kDirect);
    for (size_t p = 0; p < T.planes.size(); ++p) {
      const PlanPlane& P = T.planes[p];
      uint64_t direct = in_dev + P.payload_offset;
      if (P.codec == kCodecIdentity && !P.chunked && P.payload_len == P.plane_len && (direct & 15u) == 0)
        continue;
      const bool native = P.codec == kCodecHuffIlv || P.codec == kCodecRansIlv;
      if (native && P.chunked)  // chunk k restores at the plane offset a_k: 16-byte aligned stores
        for (size_t k = 0, a = 0; k < P.chunks.size(); a += P.chunks[k].decoded_size, ++k)
          if (a & 15u) return kUnsupported;
      scratch_off[t][p] = scratch_bytes;
      scratch_bytes = align_up(scratch_bytes + P.plane_len, 256);
      if (!native) n_jobs += P.chunked ? P.chunks.size() : 1;
    }
  }
  // the merge kernels store 16-byte pieces: a tensor whose output is not
  // 16-byte aligned is merged into scratch and copied
  std::vector<uint64_t> merge_tmp(nt, kDirect);
  for (size_t t = 0; t < nt; ++t) {
    const PlanTensor& T = plan.tensors[t];
    if (fused[t] || T.out_len == 0 || ((out_dev + T.out_offset) & 15u) == 0) continue;
    merge_tmp[t] = scratch_bytes;
    scratch_bytes = align_up(scratch_bytes + T.out_len, 256);
  }
  // planes with an inverse plane op: the op's output in scratch (the
  // decoded plane stays as it is for its CRC)
  std::vector<std::vector<uint64_t>> op_off(nt);
  for (size_t t = 0; t < nt; ++t) {
    if (fused[t]) continue;
    const PlanTensor& T = plan.tensors[t];
    op_off[t].assign(T.planes.size(), kDirect);
    for (size_t p = 0; p < T.planes.size(); ++p) {
      if (T.planes[p].op == kPlaneOpNone) continue;
      op_off[t][p] = scratch_bytes;
      scratch_bytes = align_up(scratch_bytes + T.planes[p].plane_len, 256);
    }
  }
  if (n_jobs > 0xFFFFFFFFull) return kInvalidInput;
  PTWM_HIP_TRY(ctx.planes.ensure(scratch_bytes ? scratch_bytes : 256));
  PTWM_HIP_TRY(ctx.jobs.ensure(n_jobs * sizeof(DecodeJob) + 64));
  PTWM_HIP_TRY(ctx.status.ensure(n_jobs * sizeof(uint32_t) + 64));
  PTWM_HIP_TRY(ctx.h_jobs.ensure(n_jobs * sizeof(DecodeJob) + 64));
  PTWM_HIP_TRY(ctx.h_status.ensure(n_jobs * sizeof(uint32_t) + 64));
  const uint64_t scratch_base = reinterpret_cast<uint64_t>(ctx.planes.ptr);
  DecodeJob* hj = static_cast<DecodeJob*>(ctx.h_jobs.ptr);
  std::vector<std::vector<uint64_t>> plane_addr(nt);
  size_t j = 0;
  for (size_t t = 0; t < nt; ++t) {
    if (fused[t]) continue;
    const PlanTensor& T = plan.tensors[t];
    plane_addr[t].resize(T.planes.size());
    for (size_t p = 0; p < T.planes.size(); ++p) {
      const PlanPlane& P = T.planes[p];
      if (scratch_off[t][p] == kDirect) {
        plane_addr[t][p] = in_dev + P.payload_offset;
        continue;
      }
      const uint64_t a = scratch_base + scratch_off[t][p];
      plane_addr[t][p] = a;
      if ((P.codec == kCodecHuffIlv || P.codec == kCodecRansIlv) && P.chunked) {
        uint64_t off = 0;
        for (size_t k = 0; k < P.chunks.size(); ++k) {
          IlvTensor X{};
          X.out = a + off;
          X.n = P.chunks[k].decoded_size;
          X.chain = kChainPassthrough;
          X.n_planes = 1;
          X.planes[0].base = cr.r[t][p][k].first;
          X.planes[0].len = cr.r[t][p][k].second;
          X.planes[0].coded = 1;
          X.family = P.codec == kCodecRansIlv ? kFamilyRans : kFamilyHuff;
          X.crc_first = kIlvNoCrc;
          if (X.n > 0) ilv.push_back(X);
          off += P.chunks[k].decoded_size;
        }
        continue;
      }
      if (P.codec == kCodecHuffIlv || P.codec == kCodecRansIlv) {
        if (P.plane_len == 0) continue;
        IlvTensor X{};
        X.out = a;
        X.n = P.plane_len;
        X.chain = kChainPassthrough;
        X.n_planes = 1;
        X.planes[0].base = in_dev + P.payload_offset;
        X.planes[0].len = P.payload_len;
        X.planes[0].coded = 1;
        X.family = P.codec == kCodecRansIlv ? kFamilyRans : kFamilyHuff;
        X.crc_first = kIlvNoCrc;
        ilv.push_back(X);
        continue;
      }
      if (!P.chunked) {
        DecodeJob& J = hj[j++];
        std::memset(&J, 0, sizeof(J));
        J.src = in_dev + P.payload_offset;
        J.src_len = P.payload_len;
        J.dst = a;
        J.dst_len = P.plane_len;
        J.codec = P.codec;
        J.framed = 0;
        if (P.has_state) {  // Order1ScaleAC: its state and row length
          const uint64_t sa = in_dev + P.state_offset;
          J.pad[0] = (uint32_t)sa;
          J.pad[1] = (uint32_t)(sa >> 32);
          J.pad[2] = P.state_len | (P.state_version << 24);
          J.pad[3] = P.row_len;
        }
        continue;
      }
      uint64_t dst_off = 0;
      for (size_t k = 0; k < P.chunks.size(); ++k) {
        uint64_t start = P.chunks[k].offset_in_payload;
        uint64_t end = k + 1 < P.chunks.size() ? P.chunks[k + 1].offset_in_payload : P.payload_len;
        DecodeJob& J = hj[j++];
        std::memset(&J, 0, sizeof(J));
        J.src = in_dev + P.payload_offset + start;
        J.src_len = end - start;
        J.dst = a + dst_off;
        J.dst_len = P.chunks[k].decoded_size;
        J.codec = P.codec;
        J.framed = 1;
        J.pad[3] = P.row_len;  // Order1ScaleAC: chunk frames carry the state
        dst_off += P.chunks[k].decoded_size;
      }
    }
  }
  if (j != n_jobs) return kInternal;
  hipStream_t s = ctx.stream;
  if (ctx.profile) {
    PTWM_HIP_TRY(ctx.ensure_events());
    ctx.last_ms[0] = ctx.last_ms[1] = ctx.last_ms[2] = 0;
  }
  // huff_ilv first: fused tensors straight to the output, passthrough planes to scratch
  if (!ilv.empty()) {
    if (crc_blocks) PTWM_HIP_TRY(ctx.crc_part.ensure(16ull * crc_blocks));
    int64_t rc = ilv_decode_tensors(ctx, ilv);
    if (rc != kOk) return rc;
  }
  if (ctx.profile) PTWM_HIP_TRY(hipEventRecord(ctx.ev[0], s));
  // Reference-format payloads: parallel Huffman path where it applies, exact
  // path otherwise.  Without plane ops the merges are queued right behind
  // the decode and the statuses are read once, at the end; a job decoded
  // again after that (not settled, or declined by the parallel path) has
  // its tensor merged again.
  bool any_op = false;
  for (size_t t = 0; t < nt; ++t)
    if (!fused[t])
      for (const PlanPlane& P : plan.tensors[t].planes) any_op |= P.op != kPlaneOpNone;
  ExactRun run;
  const auto complete_jobs = [&](bool& rewritten) -> int64_t {
    PTWM_HIP_TRY(hipStreamSynchronize(s));
    const int64_t rc = decode_jobs_complete(ctx, hj, n_jobs, run, rewritten);
    if (rc != kOk) return rc;
    const uint32_t* st = static_cast<const uint32_t*>(ctx.h_status.ptr);
    for (size_t k = 0; k < n_jobs; ++k)
      if (st[k] != kStOk) return kInvalidInput;
    return kOk;
  };
  if (n_jobs) {
    int64_t rc = decode_jobs_launch(ctx, hj, n_jobs, run);
    if (rc != kOk) return rc;
    if (any_op) {
      bool rewritten = false;
      rc = complete_jobs(rewritten);
      if (rc != kOk) return rc;
    }
  }
  // inverse plane ops: decoded plane -> the plane the merge reads
  std::vector<std::vector<uint64_t>> merge_addr = plane_addr;
  {
    std::vector<PlaneOpJob> ops;
    for (size_t t = 0; t < nt; ++t) {
      if (fused[t]) continue;
      const PlanTensor& T = plan.tensors[t];
      for (size_t p = 0; p < T.planes.size(); ++p) {
        const PlanPlane& P = T.planes[p];
        if (P.op == kPlaneOpNone) continue;
        merge_addr[t][p] = scratch_base + op_off[t][p];
        if (P.plane_len) ops.push_back(PlaneOpJob{plane_addr[t][p], merge_addr[t][p], P.plane_len, P.op, P.op_param, 0, 0});
      }
    }
    const int64_t rc = run_plane_ops(ctx, ops);
    if (rc != kOk) return rc;
  }
  if (ctx.profile) PTWM_HIP_TRY(hipEventRecord(ctx.ev[1], s));
  const auto launch_merges = [&]() -> int64_t {
    for (size_t t = 0; t < nt; ++t) {
      if (fused[t]) continue;
      const PlanTensor& T = plan.tensors[t];
      const uint8_t* pp[4] = {nullptr, nullptr, nullptr, nullptr};
      for (size_t p = 0; p < T.planes.size(); ++p) pp[p] = reinterpret_cast<const uint8_t*>(merge_addr[t][p]);
      uint8_t* out = reinterpret_cast<uint8_t*>(out_dev + T.out_offset);
      if (T.planes[0].plane_len == 0) continue;
      if (merge_tmp[t] == kDirect) {
        PTWM_HIP_TRY(launch_merge(T.chain, pp, T.planes[0].plane_len, out, s));
      } else {
        uint8_t* tmp = reinterpret_cast<uint8_t*>(scratch_base + merge_tmp[t]);
        PTWM_HIP_TRY(launch_merge(T.chain, pp, T.planes[0].plane_len, tmp, s));
        PTWM_HIP_TRY(hipMemcpyAsync(out, tmp, T.out_len, hipMemcpyDeviceToDevice, s));
      }
    }
    return kOk;
  };
  {
    int64_t rc = launch_merges();
    if (rc != kOk) return rc;
    if (n_jobs && !any_op) {
      bool rewritten = false;
      rc = complete_jobs(rewritten);
      if (rc != kOk) return rc;
      if (rewritten) {
        rc = launch_merges();
        if (rc != kOk) return rc;
      }
    }
  }
  if (ctx.profile) PTWM_HIP_TRY(hipEventRecord(ctx.ev[2], s));
  PTWM_HIP_TRY(hipStreamSynchronize(s));
  if (ctx.profile) {
    float a = 0, b = 0;
    PTWM_HIP_TRY(hipEventElapsedTime(&a, ctx.ev[0], ctx.ev[1]));
    PTWM_HIP_TRY(hipEventElapsedTime(&b, ctx.ev[1], ctx.ev[2]));
    ctx.last_ms[0] += a;
    ctx.last_ms[1] += b;
    ctx.last_ms[2] += a + b;
  }
  // Integrity, after every tensor is restored: CRC-32 of each decoded plane
  // (container.rs:2154-2159) and XXH64 of each restored tensor
  // (container.rs:2185-2194); a mismatch is InvalidContainer there.
  std::vector<CrcTask> crc_tasks;
  std::vector<uint32_t> crc_want;
  std::vector<FusedCrc> crc_fused;
  std::vector<uint32_t> crc_fused_want;
  std::vector<HashTask> hash_tasks;
  std::vector<uint64_t> hash_want;
  for (size_t t = 0; t < nt; ++t) {
    const PlanTensor& T = plan.tensors[t];
    if (T.has_crc && crc_first[t] != kIlvNoCrc) {
      crc_fused.push_back(FusedCrc{out_dev + T.out_offset, T.planes[0].plane_len, T.chain, crc_first[t]});
      for (const PlanPlane& P : T.planes) crc_fused_want.push_back(P.crc32);
    } else if (T.has_crc) {
      if (fused[t]) {
        crc_tasks.push_back(CrcTask{out_dev + T.out_offset, T.planes[0].plane_len, T.chain});
      } else {
        for (size_t p = 0; p < T.planes.size(); ++p)
          crc_tasks.push_back(CrcTask{plane_addr[t][p], T.planes[p].plane_len, kChainPassthrough});
      }
      for (const PlanPlane& P : T.planes) crc_want.push_back(P.crc32);
    }
    if (T.has_hash) {
      hash_tasks.push_back(HashTask{out_dev + T.out_offset, T.out_len});
      hash_want.push_back(T.xxh64);
    }
  }
  if (!crc_tasks.empty()) {
    std::vector<uint32_t> got;
    const int64_t rc = crc32_planes(ctx, crc_tasks, got);
    if (rc != kOk) return rc;
    if (got.size() != crc_want.size()) return kInternal;
    for (size_t k = 0; k < got.size(); ++k)
      if (got[k] != crc_want[k]) return kInvalidInput;
  }
  if (!crc_fused.empty()) {
    std::vector<uint32_t> got;
    const int64_t rc = crc32_fused(ctx, crc_fused, static_cast<uint32_t*>(ctx.crc_part.ptr), got);
    if (rc != kOk) return rc;
    if (got.size() != crc_fused_want.size()) return kInternal;
    for (size_t k = 0; k < got.size(); ++k)
      if (got[k] != crc_fused_want[k]) return kInvalidInput;
  }
  if (!hash_tasks.empty()) {
    std::vector<uint64_t> got;
    const int64_t rc = xxh64_buffers(ctx, hash_tasks, got);
    if (rc != kOk) return rc;
    for (size_t k = 0; k < got.size(); ++k)
      if (got[k] != hash_want[k]) return kInvalidInput;
  }
  return kOk;
}

}  // namespace ptwm
