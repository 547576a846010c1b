// integrity.hip -- CRC-32/ISO-HDLC of device buffers (decoded planes).
//
// The reference checks each decoded plane against the CRC its record carries
// (container.rs:2154-2159: crc32fast::hash of the plane bytes, crc32fast
// 1.5.0 = reflected polynomial 0xEDB88320, init and final xor 0xFFFFFFFF).
//
// GPU formulation.  A zero-initialised CRC register is linear in the data,
// and advancing it over m zero bytes multiplies it by x^(8m) mod P.  So:
//   - each workgroup takes a range of a buffer; thread t owns the 16-byte
//     pieces t, t+256, ... (coalesced dwordx4 loads) and keeps one register
//     r, relative to the end of its latest piece: r' = r x^(8 * 4096) xor
//     crc0(piece), the advance by one 4 KiB tile as four byte-sliced
//     lookups and crc0 (the zero-init CRC of the 16 bytes, slicing-by-4,
//     Kounavis & Berry 2005) independent of r, so that the serial chain per
//     piece is one round of lookups;
//   - every thread's register is moved to the range end by one GF(2)
//     multiply with x^(8d) (d = its distance to the end) and the 256 values
//     are xor-reduced: the range's zero-init CRC;
//   - a second kernel chains the ranges of each buffer the same way (Horner
//     with x^(8 range_len)) and applies init / final xor:
//     crc = ~(~0 * x^(8n) xor raw).
#include "integrity.h"

#include "chain_ops.h"
#include "crc_device.h"

#include <algorithm>
#include <vector>

namespace ptwm {

namespace {

std::vector<uint32_t> build_tables() {
  std::vector<uint32_t> tab(kCrcTabWords, 0);
  for (uint32_t i = 0; i < 256; ++i) {
    uint32_t c = i;
    for (int k = 0; k < 8; ++k) c = (c >> 1) ^ (kCrcPoly & (0u - (c & 1u)));
    tab[i] = c;
  }
  for (int k = 1; k < 4; ++k)
    for (uint32_t i = 0; i < 256; ++i) {
      const uint32_t prev = tab[256 * (k - 1) + i];
      tab[256 * k + i] = (prev >> 8) ^ tab[prev & 255u];
    }
  uint32_t* X = &tab[kCrcTabX];
  X[0] = kCrcOne >> 8;  // x^8
  for (int k = 1; k < 64; ++k) X[k] = gf2_mulmod(X[k - 1], X[k - 1]);
  const uint32_t adv = xpow8(kCrcTile, X);
  for (int k = 0; k < 4; ++k)
    for (uint32_t b = 0; b < 256; ++b) tab[kCrcTabS + 256 * k + b] = gf2_mulmod(b << (8 * k), adv);
  for (uint32_t t = 0; t < kCrcThreads; ++t) tab[kCrcTabK + t] = xpow8((uint64_t)kCrcPiece * (kCrcThreads - 1 - t), X);
  const uint32_t adv1k = xpow8(1024, X);
  for (int k = 0; k < 4; ++k)
    for (uint32_t b = 0; b < 256; ++b) tab[kCrcTabS1024 + 256 * k + b] = gf2_mulmod(b << (8 * k), adv1k);
  for (uint32_t l = 0; l < 64; ++l) tab[kCrcTabK64 + l] = xpow8(16ull * (63 - l), X);
  return tab;
}

__device__ __forceinline__ uint32_t block_xor(uint32_t v, uint32_t* red) {
  for (int d = 32; d >= 1; d >>= 1) v ^= __shfl_xor(v, d, 64);
  if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return red[0] ^ red[1] ^ red[2] ^ red[3];
}

// Zero-init CRC of each range, relative to the range's end, for every plane
// of the range, to part[4 * r + plane] with r = slot[range] (slot null: r =
// range).  A range is a run of whole elements of one buffer; with kChain =
// passthrough the buffer is a plane itself, otherwise a restored tensor
// whose plane bytes are re-derived by the (bijective) forward chain.
template <uint32_t kChain>
__global__ void __launch_bounds__(256) crc_range_kernel(const CrcRange* __restrict__ ranges,
                                                        const uint32_t* __restrict__ gtab,
                                                        uint32_t* __restrict__ part,
                                                        const uint32_t* __restrict__ slot) {
  constexpr int kNp = kChain == kChainIeee16Split2 ? 2 : kChain == kChainIeee32Split4 ? 4 : 1;
  constexpr int kRatio = kNp;  // tensor bytes per plane byte for these chains
  __shared__ uint32_t tab[kCrcTabK];  // T0..T3, S0..S3
  __shared__ uint32_t red[4];
  const uint32_t t = threadIdx.x;
  for (uint32_t i = t; i < kCrcTabK; i += kCrcThreads) tab[i] = gtab[i];
  const CrcRange R = ranges[blockIdx.x];
  __syncthreads();
  const uint32_t* T = tab;
  const uint32_t* S = tab + kCrcTabS;
  const uint64_t full = R.n / kCrcTile, tail = R.n % kCrcTile;
  const u32x4* p = reinterpret_cast<const u32x4*>(R.src) + (uint64_t)t * kRatio;
  uint32_t acc[kNp];
#pragma unroll
  for (int j = 0; j < kNp; ++j) acc[j] = 0;
  auto step = [&](uint64_t k) {
    u32x4 v[kRatio], pl[kNp];
#pragma unroll
    for (int h = 0; h < kRatio; ++h) v[h] = g_ld_nt16(reinterpret_cast<uint64_t>(p + k * kCrcThreads * kRatio + h));
    forward16<kChain>(v, pl);
#pragma unroll
    for (int j = 0; j < kNp; ++j) acc[j] = sliced(S, acc[j]) ^ crc_piece(T, 0u, pl[j]);
  };
  // four tiles per iteration, their loads issued before any lookup
  constexpr int kU = 4;
  uint64_t k = 0;
  for (; k + kU <= full; k += kU) {
    u32x4 v[kU][kRatio];
#pragma unroll
    for (int u = 0; u < kU; ++u)
#pragma unroll
      for (int h = 0; h < kRatio; ++h)
        v[u][h] = g_ld_nt16(reinterpret_cast<uint64_t>(p + (k + u) * kCrcThreads * kRatio + h));
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      u32x4 pl[kNp];
      forward16<kChain>(v[u], pl);
#pragma unroll
      for (int j = 0; j < kNp; ++j) acc[j] = sliced(S, acc[j]) ^ crc_piece(T, 0u, pl[j]);
    }
  }
  for (; k < full; ++k) step(k);
  if (tail == 0) {
    if (full) {
      const uint32_t K = gtab[kCrcTabK + t];
#pragma unroll
      for (int j = 0; j < kNp; ++j) acc[j] = gf2_mulmod(acc[j], K);
    }
  } else {
    // the last, partial tile: thread t's piece may be whole, cut, or absent
    const uint64_t base = full * kCrcTile + (uint64_t)kCrcPiece * t;
    uint64_t end = full ? base - kCrcTile + kCrcPiece : 0;
    bool any = full != 0;
    if (base + kCrcPiece <= R.n) {
      step(full);
      end = base + kCrcPiece;
      any = true;
    } else if (base < R.n) {
      // the register advanced over the gap before this piece
      const uint32_t gap = full ? xpow8(kCrcTile - kCrcPiece, gtab + kCrcTabX) : 0u;
#pragma unroll
      for (int j = 0; j < kNp; ++j) {
        uint32_t c = gf2_mulmod(acc[j], gap);
        for (uint64_t i = base; i < R.n; ++i) c = T[(c ^ forward_byte<kChain>(R.src, i, j)) & 255u] ^ (c >> 8);
        acc[j] = c;
      }
      end = R.n;
      any = true;
    }
    if (any) {
      const uint32_t K = xpow8(R.n - end, gtab + kCrcTabX);
#pragma unroll
      for (int j = 0; j < kNp; ++j) acc[j] = gf2_mulmod(acc[j], K);
    }
  }
#pragma unroll
  for (int j = 0; j < kNp; ++j) {
    const uint32_t v = block_xor(acc[j], red);
    if (t == 0) part[4ull * (slot ? slot[blockIdx.x] : blockIdx.x) + j] = v;
    __syncthreads();
  }
}

// Chains the ranges of one plane (blockIdx.x), applies init / final xor,
// writes the plane's CRC.  Multiplying by the whole-range shift s_full is
// linear in the multiplicand, so it runs as four byte-sliced lookups into
// tables of (v << 8k) * s_full built in LDS first.
__global__ void __launch_bounds__(256) crc_combine_kernel(const CrcPlane* __restrict__ planes,
                                                          const uint32_t* __restrict__ part,
                                                          const uint32_t* __restrict__ gtab,
                                                          uint32_t* __restrict__ crc_out) {
  __shared__ uint32_t red[4];
  __shared__ uint32_t mt[4][256];
  const CrcPlane B = planes[blockIdx.x];
  const uint32_t* X = gtab + kCrcTabX;
  const uint32_t t = threadIdx.x;
  const uint32_t s_full = xpow8(B.range_len, X);
  static_assert(kCrcThreads == 256, "one table entry per thread and slice");
#pragma unroll
  for (uint32_t k = 0; k < 4; ++k) mt[k][t] = gf2_mulmod(t << (8 * k), s_full);
  __syncthreads();
  const uint32_t q = (B.n_ranges + kCrcThreads - 1) / kCrcThreads;
  const uint32_t r0 = std::min(B.n_ranges, t * q), r1 = std::min(B.n_ranges, r0 + q);
  uint32_t acc = 0;
  if (r0 < r1) {
    const uint64_t last_len = B.n - (uint64_t)(B.n_ranges - 1) * B.range_len;
    for (uint32_t r = r0; r < r1; ++r) {
      const uint32_t x = r + 1 == B.n_ranges ? gf2_mulmod(acc, xpow8(last_len, X))
                                             : mt[0][acc & 255u] ^ mt[1][(acc >> 8) & 255u] ^
                                                   mt[2][(acc >> 16) & 255u] ^ mt[3][acc >> 24];
      acc = x ^ part[4ull * (B.first_range + r) + B.plane];
    }
    const uint64_t end = r1 == B.n_ranges ? B.n : (uint64_t)r1 * B.range_len;
    acc = gf2_mulmod(acc, xpow8(B.n - end, X));
  }
  acc = block_xor(acc, red);
  if (t == 0) crc_out[blockIdx.x] = ~(gf2_mulmod(0xFFFFFFFFu, xpow8(B.n, X)) ^ acc);
}

int chain_np(uint32_t chain) { return chain == kChainIeee16Split2 ? 2 : chain == kChainIeee32Split4 ? 4 : 1; }

// c: 0 = IEEE16 split2, 1 = IEEE32 split4, 2 = passthrough
hipError_t launch_crc_ranges(int c, uint32_t cnt, const CrcRange* r, const uint32_t* gtab, uint32_t* part,
                             const uint32_t* slot, hipStream_t s) {
  const dim3 g(cnt), b(kCrcThreads);
  if (c == 0) hipLaunchKernelGGL(crc_range_kernel<kChainIeee16Split2>, g, b, 0, s, r, gtab, part, slot);
  if (c == 1) hipLaunchKernelGGL(crc_range_kernel<kChainIeee32Split4>, g, b, 0, s, r, gtab, part, slot);
  if (c == 2) hipLaunchKernelGGL(crc_range_kernel<kChainPassthrough>, g, b, 0, s, r, gtab, part, slot);
  return hipGetLastError();
}

}  // namespace

bool crc_chain_supported(uint32_t chain) {
  return chain == kChainIeee16Split2 || chain == kChainIeee32Split4 || chain == kChainPassthrough;
}

int64_t crc_tables(DevCtx& ctx, const uint32_t** tab) {
  if (!ctx.crc_tab_ready) {
    const std::vector<uint32_t> t = build_tables();
    PTWM_HIP_TRY(ctx.crc_tab.ensure(t.size() * 4));
    PTWM_HIP_TRY(hipMemcpyAsync(ctx.crc_tab.ptr, t.data(), t.size() * 4, hipMemcpyHostToDevice, ctx.stream));
    PTWM_HIP_TRY(hipStreamSynchronize(ctx.stream));
    ctx.crc_tab_ready = true;
  }
  *tab = static_cast<const uint32_t*>(ctx.crc_tab.ptr);
  return kOk;
}

int64_t crc32_combine(DevCtx& ctx, const std::vector<CrcPlane>& planes, const uint32_t* d_part,
                      std::vector<uint32_t>& crcs) {
  crcs.assign(planes.size(), 0);
  if (planes.empty()) return kOk;
  hipStream_t s = ctx.stream;
  const uint32_t* gtab = nullptr;
  if (int64_t rc = crc_tables(ctx, &gtab); rc != kOk) return rc;
  const size_t np = planes.size();
  PTWM_HIP_TRY(ctx.crc_comb.ensure(np * (sizeof(CrcPlane) + 4) + 64));
  CrcPlane* d_planes = static_cast<CrcPlane*>(ctx.crc_comb.ptr);
  uint32_t* d_out = reinterpret_cast<uint32_t*>(d_planes + np);
  PTWM_HIP_TRY(hipMemcpyAsync(d_planes, planes.data(), np * sizeof(CrcPlane), hipMemcpyHostToDevice, s));
  for (size_t p0 = 0; p0 < np; p0 += 65535) {
    const uint32_t cnt = (uint32_t)std::min<size_t>(65535, np - p0);
    hipLaunchKernelGGL(crc_combine_kernel, dim3(cnt), dim3(kCrcThreads), 0, s, d_planes + p0, d_part, gtab, d_out + p0);
    PTWM_HIP_TRY(hipGetLastError());
  }
  PTWM_HIP_TRY(hipMemcpyAsync(crcs.data(), d_out, np * 4, hipMemcpyDeviceToHost, s));
  PTWM_HIP_TRY(hipStreamSynchronize(s));
  return kOk;
}

int64_t crc32_fused(DevCtx& ctx, const std::vector<FusedCrc>& tensors, uint32_t* d_part, std::vector<uint32_t>& crcs) {
  crcs.clear();
  if (tensors.empty()) return kOk;
  hipStream_t s = ctx.stream;
  const uint32_t* gtab = nullptr;
  if (int64_t rc = crc_tables(ctx, &gtab); rc != kOk) return rc;
  // the partial last blocks, by chain (the decode wrote the whole ones)
  const uint32_t chains[3] = {kChainIeee16Split2, kChainIeee32Split4, kChainPassthrough};
  std::vector<CrcRange> ranges;
  std::vector<uint32_t> slots;
  uint32_t first[4] = {0, 0, 0, 0};
  std::vector<CrcPlane> planes;
  for (int c = 0; c < 3; ++c) {
    first[c] = (uint32_t)ranges.size();
    for (const FusedCrc& f : tensors) {
      if (f.chain != chains[c] || f.n % kFusedCrcBlock == 0) continue;
      const uint64_t nb = (f.n + kFusedCrcBlock - 1) / kFusedCrcBlock;
      const uint64_t b0 = (nb - 1) * kFusedCrcBlock;
      if (f.out & 15u) return kInternal;
      ranges.push_back(CrcRange{f.out + b0 * (uint64_t)chain_np(f.chain), f.n - b0});
      slots.push_back((uint32_t)(f.first_block + nb - 1));
    }
  }
  first[3] = (uint32_t)ranges.size();
  for (const FusedCrc& f : tensors) {
    if (!crc_chain_supported(f.chain) || f.n == 0) return kInternal;
    const uint32_t nb = (uint32_t)((f.n + kFusedCrcBlock - 1) / kFusedCrcBlock);
    for (int j = 0; j < chain_np(f.chain); ++j)
      planes.push_back(CrcPlane{f.n, kFusedCrcBlock, f.first_block, nb, (uint32_t)j});
  }
  const size_t nr = ranges.size();
  if (nr) {
    PTWM_HIP_TRY(ctx.crc_args.ensure(nr * (sizeof(CrcRange) + 4) + 64));
    CrcRange* d_ranges = static_cast<CrcRange*>(ctx.crc_args.ptr);
    uint32_t* d_slots = reinterpret_cast<uint32_t*>(d_ranges + nr);
    PTWM_HIP_TRY(hipMemcpyAsync(d_ranges, ranges.data(), nr * sizeof(CrcRange), hipMemcpyHostToDevice, s));
    PTWM_HIP_TRY(hipMemcpyAsync(d_slots, slots.data(), nr * 4, hipMemcpyHostToDevice, s));
    for (int c = 0; c < 3; ++c) {
      const uint32_t cnt = first[c + 1] - first[c];
      if (cnt) PTWM_HIP_TRY(launch_crc_ranges(c, cnt, d_ranges + first[c], gtab, d_part, d_slots + first[c], s));
    }
  }
  return crc32_combine(ctx, planes, d_part, crcs);
}

int64_t crc32_planes(DevCtx& ctx, const std::vector<CrcTask>& tasks, std::vector<uint32_t>& crcs) {
  crcs.clear();
  if (tasks.empty()) return kOk;
  hipStream_t s = ctx.stream;
  const uint32_t* tabs = nullptr;
  if (int64_t rc = crc_tables(ctx, &tabs); rc != kOk) return rc;
  // Range length (plane bytes): a multiple of the 4 KiB tile, sized so the
  // whole batch makes about 16 workgroups per CU.
  uint64_t total = 0;
  for (const CrcTask& k : tasks) {
    if (!crc_chain_supported(k.chain)) return kInternal;
    if (k.n && (k.src & 15u)) return kInternal;  // callers pass 16-byte aligned buffers
    total += k.n * (uint64_t)chain_np(k.chain);
  }
  const uint64_t cus = ctx.cu_count > 0 ? (uint64_t)ctx.cu_count : 256;
  uint64_t rl = (total / (cus * 16) + kCrcTile - 1) / kCrcTile * kCrcTile;
  rl = std::max<uint64_t>(rl, 16 * kCrcTile);
  rl = std::min<uint64_t>(rl, 1ull << 30);
  // ranges grouped by chain (one launch per chain), planes in task order
  const uint32_t chains[3] = {kChainIeee16Split2, kChainIeee32Split4, kChainPassthrough};
  std::vector<CrcRange> ranges;
  std::vector<CrcPlane> planes;
  uint32_t first[4] = {0, 0, 0, 0};
  std::vector<uint32_t> task_plane0(tasks.size(), 0);
  for (int c = 0; c < 3; ++c) {
    first[c] = (uint32_t)ranges.size();
    for (size_t i = 0; i < tasks.size(); ++i) {
      const CrcTask& k = tasks[i];
      if (k.chain != chains[c]) continue;
      const uint32_t fr = (uint32_t)ranges.size();
      const uint64_t ratio = (uint64_t)chain_np(k.chain);
      for (uint64_t o = 0; o < k.n; o += rl) ranges.push_back(CrcRange{k.src + o * ratio, std::min(rl, k.n - o)});
      (void)fr;
    }
  }
  first[3] = (uint32_t)ranges.size();
  // planes: walk tasks again in order, matching the range numbering above
  {
    std::vector<uint32_t> next(3);
    for (int c = 0; c < 3; ++c) next[c] = first[c];
    for (size_t i = 0; i < tasks.size(); ++i) {
      const CrcTask& k = tasks[i];
      const int c = k.chain == kChainIeee16Split2 ? 0 : k.chain == kChainIeee32Split4 ? 1 : 2;
      const uint32_t nr = (uint32_t)((k.n + rl - 1) / rl);
      task_plane0[i] = (uint32_t)planes.size();
      for (int j = 0; j < chain_np(k.chain); ++j)
        planes.push_back(CrcPlane{k.n, (uint32_t)rl, next[c], nr, (uint32_t)j});
      next[c] += nr;
    }
  }
  const size_t nr = ranges.size(), np = planes.size();
  PTWM_HIP_TRY(ctx.crc_args.ensure(nr * sizeof(CrcRange) + np * sizeof(CrcPlane) + (4 * nr + np) * 4 + 64));
  uint8_t* base = static_cast<uint8_t*>(ctx.crc_args.ptr);
  CrcRange* d_ranges = reinterpret_cast<CrcRange*>(base);
  CrcPlane* d_planes = reinterpret_cast<CrcPlane*>(base + nr * sizeof(CrcRange));
  uint32_t* d_part = reinterpret_cast<uint32_t*>(base + nr * sizeof(CrcRange) + np * sizeof(CrcPlane));
  uint32_t* d_out = d_part + 4 * nr;
  if (nr) PTWM_HIP_TRY(hipMemcpyAsync(d_ranges, ranges.data(), nr * sizeof(CrcRange), hipMemcpyHostToDevice, s));
  PTWM_HIP_TRY(hipMemcpyAsync(d_planes, planes.data(), np * sizeof(CrcPlane), hipMemcpyHostToDevice, s));
  const uint32_t* gtab = tabs;
  for (int c = 0; c < 3; ++c) {
    const uint32_t cnt = first[c + 1] - first[c];
    if (!cnt) continue;
    const CrcRange* r = d_ranges + first[c];
    uint32_t* pp = d_part + 4ull * first[c];
    PTWM_HIP_TRY(launch_crc_ranges(c, cnt, r, gtab, pp, nullptr, s));
  }
  for (size_t p0 = 0; p0 < np; p0 += 65535) {
    const uint32_t cnt = (uint32_t)std::min<size_t>(65535, np - p0);
    hipLaunchKernelGGL(crc_combine_kernel, dim3(cnt), dim3(kCrcThreads), 0, s, d_planes + p0, d_part, gtab, d_out + p0);
    PTWM_HIP_TRY(hipGetLastError());
  }
  crcs.assign(np, 0);
  PTWM_HIP_TRY(hipMemcpyAsync(crcs.data(), d_out, np * 4, hipMemcpyDeviceToHost, s));
  PTWM_HIP_TRY(hipStreamSynchronize(s));
  return kOk;
}

}  // namespace ptwm
