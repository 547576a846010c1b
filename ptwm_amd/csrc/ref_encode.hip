// ref_encode.hip -- GPU encoder for the reference's Huffman and rANS plane
// payloads, byte-identical to the reference encoder.
//
// Payload framing: codecs/huffman.rs:37-87 and codecs/rans.rs:38-94
// ([00] empty, [00]+raw when not beneficial, [01][orig_len u32][blob]);
// blobs: entropy/huffman/compress.rs:9-103 (weights header, jump table,
// four backward bitstreams over split_four segments) and
// entropy/rans/compress.rs:128-260 (frequency header, jump table, four
// streams [x_final u32][renorm bytes in decoder order]).
//
// One call encodes a batch of jobs (each one payload: a whole plane or one
// chunk of a chunked plane):
//   1. histogram per job (ref_hist_kernel);
//   2. host: code tables per job (huffman_host.cpp: the reference tree,
//      canonical codes and weights header; rANS: normalize_freqs and the
//      EncSymbol reciprocal parameters of rans/compress.rs:35-122);
//   3. Huffman: bits per segment from the segment's histogram and the code
//      lengths (the histograms are taken per split_four segment); rANS:
//      each segment encoded by one lane into scratch (ref_rans_kernel; a
//      segment's state chain is serial by construction, 64 segments run
//      per wavefront);
//   4. host: payload sizes, coded-or-raw decisions, output layout;
//   5. Huffman segments packed in parallel: every symbol's bit offset is a
//      prefix sum of code lengths, so each segment is cut into slices of
//      kSliceSyms symbols, the bits of every slice summed
//      (ref_huf_slice_bits_kernel) and scanned per segment
//      (ref_huf_slice_scan_kernel), and every slice packed from its offset
//      by its own workgroup (ref_huf_pack_kernel); then headers, streams
//      and raw fallbacks placed by one gather launch of 64 KiB pieces
//      (ref_copy_kernel).
#include "ref_encode.h"

#include <algorithm>
#include <cstring>

#include "huffman_host.h"

namespace ptwm {

namespace {

constexpr uint32_t kRansProbBits = 11;
constexpr uint32_t kRansScale = 1u << kRansProbBits;
constexpr uint32_t kRansL = 1u << 23;

__device__ __forceinline__ uint8_t gbyte(uint64_t a) {
  return *(const __attribute__((address_space(1))) uint8_t*)(uintptr_t)a;
}

// atomic OR into global memory (not a flat atomic: see g_ld)
__device__ __forceinline__ void or_global(uint32_t* p, uint32_t v) {
  __hip_atomic_fetch_or((__attribute__((address_space(1))) uint32_t*)(uintptr_t)p, v, __ATOMIC_RELAXED,
                        __HIP_MEMORY_SCOPE_AGENT);
}

// 256-bin histogram per job (blockIdx.y); any source alignment.
__global__ void __launch_bounds__(256) ref_hist_kernel(const RefJobDev* __restrict__ jobs, uint32_t* __restrict__ hist) {
  __shared__ uint32_t h[4][256];
  const RefJobDev J = jobs[blockIdx.y];
  const uint32_t t = threadIdx.x, wave = t >> 6;
  for (uint32_t i = t; i < 1024; i += 256) (&h[0][0])[i] = 0;
  __syncthreads();
  const uint64_t head = J.n == 0 ? 0 : std::min<uint64_t>(J.n, (16 - (J.src & 15)) & 15);
  const uint64_t nvec = (J.n - head) / 16;
  const uint64_t stride = (uint64_t)gridDim.x * 256u;
  const u32x4* v = reinterpret_cast<const u32x4*>(J.src + head);
  for (uint64_t i = (uint64_t)blockIdx.x * 256u + t; i < nvec; i += stride) {
    const u32x4 x = g_ld_nt16(reinterpret_cast<uint64_t>(v + i));
    const uint32_t xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int b = 0; b < 4; ++b) atomicAdd(&h[wave][(xs[k] >> (8 * b)) & 0xFF], 1u);
  }
  if (blockIdx.x == 0) {
    for (uint64_t i = t; i < head; i += 256) atomicAdd(&h[wave][gbyte(J.src + i)], 1u);
    for (uint64_t i = head + nvec * 16 + t; i < J.n; i += 256) atomicAdd(&h[wave][gbyte(J.src + i)], 1u);
  }
  __syncthreads();
  const uint32_t s = h[0][t] + h[1][t] + h[2][t] + h[3][t];
  if (s) atomicAdd(&hist[256u * blockIdx.y + t], s);
}

// Huffman: total code bits of each slice.  The slice's bytes are read as the
// aligned words that hold them, one word per thread per step.
__global__ void __launch_bounds__(256) ref_huf_slice_bits_kernel(const RefSegDev* __restrict__ segs,
                                                                 const RefSliceDev* __restrict__ slices,
                                                                 const uint32_t* __restrict__ codes,
                                                                 unsigned long long* __restrict__ slice_bits) {
  __shared__ uint8_t len[256];
  __shared__ unsigned long long part[4];
  const RefSliceDev L = slices[blockIdx.x];
  const RefSegDev S = segs[L.seg];
  const uint32_t t = threadIdx.x;
  len[t] = (uint8_t)(codes[256u * S.table + t] >> 16);
  __syncthreads();
  const uint64_t b0 = S.src + L.sym0, b1 = b0 + L.n, a0 = b0 & ~3ull;
  unsigned long long bits = 0;
  for (uint64_t a = a0 + 4ull * t; a < b1; a += 1024) {
    const uint32_t w = g_ld<uint32_t>(a);
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k)
      if (a + k >= b0 && a + k < b1) bits += len[(w >> (8 * k)) & 0xFFu];
  }
  for (int d = 32; d >= 1; d >>= 1) bits += __shfl_down(bits, d, 64);
  if ((t & 63u) == 0) part[t >> 6] = bits;
  __syncthreads();
  if (t == 0) slice_bits[blockIdx.x] = part[0] + part[1] + part[2] + part[3];
}

// Exclusive scan of each segment's slice bits (workgroup g: the slices
// [first[g], first[g + 1])), in place: each slice's starting bit.
__global__ void __launch_bounds__(256) ref_huf_slice_scan_kernel(const uint32_t* __restrict__ first,
                                                                 unsigned long long* __restrict__ slice_bits) {
  __shared__ unsigned long long wsum[4];
  const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
  const uint32_t s0 = first[blockIdx.x], s1 = first[blockIdx.x + 1];
  unsigned long long carry = 0;
  for (uint32_t b = s0; b < s1; b += 256) {
    const uint32_t i = b + t;
    const unsigned long long v = i < s1 ? slice_bits[i] : 0ull;
    unsigned long long incl = v;
#pragma unroll
    for (uint32_t d = 1; d < 64; d <<= 1) {
      const unsigned long long o = __shfl_up(incl, d, 64);
      if (lane >= d) incl += o;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    unsigned long long before = 0, tot = 0;
    for (uint32_t w = 0; w < 4; ++w) {
      if (w < wave) before += wsum[w];
      tot += wsum[w];
    }
    if (i < s1) slice_bits[i] = carry + before + incl - v;
    carry += tot;
    __syncthreads();
  }
}

// Huffman: pack one segment's codes (bit-reversed canonical codes,
// LSB-first, bitstream.rs:22-50) straight into their final byte order.  The
// logical stream P (bit k = bit k % 8 of byte k / 8) is stored reversed
// (S[m-1-i] = P[i]); in the segment's word-aligned scratch area of W words
// whose last m bytes are S, logical word w is the byte-swapped word W-1-w.
// One workgroup per slice (slice_off: the slice's first bit).  Each pass
// covers 256 x kPackPerThread symbols: every thread reads its symbols as
// the aligned words that hold them, a workgroup scan gives each thread its
// bit offset, the pass's words are assembled in LDS (OR), and written out:
// the pass's first and last word with a global OR (they may be shared with
// the neighbouring pass or slice; the area starts zeroed), the others with
// plain stores.
constexpr uint32_t kPackPerThread = 8;
constexpr uint32_t kPackWords = (256u * kPackPerThread * 11u + 31u) / 32u + 2u;
__global__ void __launch_bounds__(256) ref_huf_pack_kernel(const RefSegDev* __restrict__ segs,
                                                           const RefSliceDev* __restrict__ slices,
                                                           const unsigned long long* __restrict__ slice_off,
                                                           const uint32_t* __restrict__ codes,
                                                           uint32_t* __restrict__ scratch) {
  __shared__ uint32_t code[256];
  __shared__ uint32_t wave_sum[4];
  __shared__ uint32_t asm_w[kPackWords];
  const RefSliceDev L = slices[blockIdx.x];
  const RefSegDev S = segs[L.seg];
  const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
  code[t] = codes[256u * S.table + t];
  unsigned long long base = slice_off[blockIdx.x];
  uint32_t* area = scratch + S.scratch_word;
  const uint64_t W = S.words;
  const uint64_t src = S.src + L.sym0, end = src + L.n;
  __syncthreads();
  for (uint64_t pass = 0; pass < L.n; pass += 256ull * kPackPerThread) {
    for (uint32_t k = t; k < kPackWords; k += 256) asm_w[k] = 0;
    // this thread's symbols: bytes [a, a + 8) of the slice, from the three
    // aligned words that hold them (a word is read only if it starts
    // before the slice's end, so it holds one of the slice's bytes)
    const uint64_t a = src + pass + (uint64_t)t * kPackPerThread;
    const uint64_t aw = a & ~3ull;
    const uint32_t sh = (uint32_t)(a & 3u);
    uint32_t w[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) w[k] = aw + 4u * k < end ? g_ld<uint32_t>(aw + 4u * k) : 0u;
    const uint32_t lo = __builtin_amdgcn_alignbyte(w[1], w[0], sh), hi = __builtin_amdgcn_alignbyte(w[2], w[1], sh);
    uint32_t sym_code[kPackPerThread];
    uint32_t bits = 0;
#pragma unroll
    for (uint32_t k = 0; k < kPackPerThread; ++k) {
      const uint32_t b = ((k < 4 ? lo : hi) >> (8 * (k & 3))) & 0xFFu;
      sym_code[k] = a + k < end ? code[b] : 0u;
      bits += sym_code[k] >> 16;
    }
    // exclusive prefix of bits over the workgroup
    uint32_t incl = bits;
#pragma unroll
    for (uint32_t d = 1; d < 64; d <<= 1) {
      const uint32_t o = __shfl_up(incl, d, 64);
      if (lane >= d) incl += o;
    }
    if (lane == 63) wave_sum[wave] = incl;
    __syncthreads();
    uint32_t before = 0, pass_bits = 0;
    for (uint32_t v = 0; v < 4; ++v) {
      if (v < wave) before += wave_sum[v];
      pass_bits += wave_sum[v];
    }
    // LDS word j holds the pass's logical word (base >> 5) + j
    const uint32_t b0 = (uint32_t)(base & 31u);
    uint32_t off = b0 + before + (incl - bits);
    uint32_t j = off >> 5, fill = off & 31u;
    uint64_t acc = 0;
#pragma unroll
    for (uint32_t k = 0; k < kPackPerThread; ++k) {
      acc |= (uint64_t)(sym_code[k] & 0xFFFFu) << fill;
      fill += sym_code[k] >> 16;
      if (fill >= 32) {
        atomicOr(&asm_w[j], (uint32_t)acc);
        acc >>= 32;
        fill -= 32;
        ++j;
      }
    }
    if (fill) atomicOr(&asm_w[j], (uint32_t)acc);
    __syncthreads();
    const uint32_t nw = (b0 + pass_bits + 31u) >> 5;
    const uint64_t w0 = base >> 5;
    for (uint32_t k = t; k < nw; k += 256) {
      uint32_t* dst = area + (W - 1 - (w0 + k));
      const uint32_t v = __builtin_bswap32(asm_w[k]);
      if (k == 0 || k + 1 == nw) or_global(dst, v);
      else g_st<uint32_t>(reinterpret_cast<uint64_t>(dst), v);
    }
    base += pass_bits;
    __syncthreads();
  }
}

// rANS: one lane encodes one segment backward (encode_stream_into,
// rans/compress.rs:140-185) into its scratch area: [x_final u32 LE][renorm
// bytes in emission order]; seg_len = 4 + renorm bytes.  Table entries per
// symbol: {rcp, bias, cmpl | shift << 24, freq << 20}.
//
// The state chain is serial by the format, so a step is kept short:
// - the segment's symbols arrive as 16-byte aligned blocks, walked from the
//   last to the first, each loaded four blocks ahead (a step takes exactly
//   one symbol, so the schedule is fixed; aligned blocks that hold a byte of
//   the segment never cross a page, so reading them whole is in bounds);
// - the tables of the workgroup's jobs sit in LDS, and a block's sixteen
//   entries, which depend on its symbols only, are read before its steps;
// - x sheds its low byte while x >= freq << 20 (at most twice): both tests
//   and both shifts run side by side, and the two low bytes of x go to the
//   lane's LDS output buffer every step (a byte not shed is overwritten by
//   the next step's); the buffer's whole words go to the scratch after each
//   block as a fixed nine word stores.
constexpr uint32_t kRansEncLanes = 64;                    // segments per workgroup
constexpr uint32_t kRansEncJobs = kRansEncLanes / 4 + 1;  // job tables a workgroup can span
constexpr uint32_t kRansEncOut = 48;                      // output buffer bytes per lane (3 + 32, words)
constexpr uint64_t kRansEncSlack = 64;                    // scratch bytes past a segment's stream the flush may write

__global__ void __launch_bounds__(kRansEncLanes) ref_rans_kernel(const RefSegDev* __restrict__ segs, uint32_t n_segs,
                                                                 const uint4* __restrict__ tables,
                                                                 uint8_t* __restrict__ scratch,
                                                                 unsigned long long* __restrict__ seg_len) {
  __shared__ uint4 tab[kRansEncJobs][257];  // + the identity entry
  __shared__ __align__(16) uint8_t obuf[kRansEncLanes * kRansEncOut];
  const uint32_t s0 = blockIdx.x * kRansEncLanes, lane = threadIdx.x;
  const uint32_t s = s0 + lane;
  const uint32_t last = min(n_segs, s0 + kRansEncLanes) - 1;
  // A job's four segments are consecutive, so the workgroup's segments form
  // runs of one job each (at most kRansEncJobs): run r's table goes to tab[r].
  const uint32_t job = segs[min(s, last)].table;
  const uint32_t prev_job = (uint32_t)__shfl_up((int)job, 1, 64);
  const uint64_t starts = __ballot(lane == 0 || prev_job != job);
  const uint32_t slot = (uint32_t)__popcll(starts & ((2ull << lane) - 1)) - 1;
  uint64_t rest = starts;
  for (uint32_t r = 0; rest; ++r) {
    const uint32_t at = (uint32_t)__builtin_ctzll(rest);
    rest &= rest - 1;
    const uint32_t jr = (uint32_t)__builtin_amdgcn_readlane((int)job, at);
    for (uint32_t i = lane; i < 256; i += kRansEncLanes) tab[r][i] = tables[256ull * jr + i];
    // identity: rcp 0, bias 0, cmpl 0, no byte shed below 2^32 - 1
    if (lane == 0) tab[r][256] = make_uint4(0u, 0u, 0u, 0xFFFFFFFFu);
  }
  __syncthreads();
  if (s >= n_segs) return;
  const RefSegDev S = segs[s];
  const uint4* const T = tab[slot];
  const uint64_t out = reinterpret_cast<uint64_t>(scratch + S.scratch_byte);
  uint8_t* const ob = obuf + lane * kRansEncOut;
  uint32_t x = kRansL;
  uint64_t nb = 4;  // stream bytes stored after x_final
  uint32_t E = 0;   // bytes in ob
  if (S.n) {
    const uint64_t first = S.src, end = S.src + S.n;  // symbols [first, end)
    const uint64_t b_lo = first & ~15ull;
    uint64_t blk = (end - 1) & ~15ull;  // block holding the last symbol
    // one step (rans/compress.rs:150-167)
    auto step = [&](const uint4 e) {
      const bool n1 = x >= e.w, n2 = (x >> 8) >= e.w;
      const uint32_t xs = n2 ? x >> 16 : n1 ? x >> 8 : x;
      ob[E] = (uint8_t)x;  // byte stores: a 16-bit LDS store needs an even address
      ob[E + 1] = (uint8_t)(x >> 8);
      E += (uint32_t)n1 + (uint32_t)n2;
      const uint32_t q = __umulhi(xs, e.x) >> (e.z >> 24);
      x = xs + e.y + __umul24(q, e.z);
    };
    // One 16-symbol block, last symbol first.  In the segment's first and
    // last blocks, positions outside the segment take the identity entry.
    // Every symbol of the data has a nonzero frequency (the table is
    // normalised from the same bytes' histogram).
    auto block = [&](const u32x4 v, uint64_t at) {
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
      uint4 e[16];
      if (at >= first && at + 16 <= end) {
#pragma unroll
        for (int i = 0; i < 16; ++i) e[i] = T[(w[i >> 2] >> (8 * (i & 3))) & 0xFFu];
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const uint64_t a = at + (uint64_t)i;
          e[i] = T[a >= first && a < end ? (w[i >> 2] >> (8 * (i & 3))) & 0xFFu : 256u];
        }
      }
#pragma unroll
      for (int i = 15; i >= 0; --i) step(e[i]);
      // whole words of the buffer to the scratch (nine stores: at most 3 + 32
      // bytes; words past the last whole one are rewritten by later flushes)
      const uint32_t* o32 = reinterpret_cast<const uint32_t*>(ob);
#pragma unroll
      for (int k = 0; k < 9; ++k) g_st<uint32_t>(out + nb + 4 * k, o32[k]);
      const uint32_t nd = E >> 2;
      nb += 4 * nd;
      *reinterpret_cast<uint32_t*>(ob) = o32[nd];
      E &= 3;
    };
    // four blocks in flight, each slot refilled with the block four below
    // it; every load is issued (below the segment's first block it reads
    // that block again) so that the wait before a block's use counts the
    // loads and stores issued after it
    auto at_or_lo = [&](uint64_t a) { return a >= b_lo + 64 ? a - 64 : b_lo; };
    u32x4 r0 = g_ld<u32x4>(blk);
    u32x4 r1 = g_ld<u32x4>(blk >= b_lo + 16 ? blk - 16 : b_lo);
    u32x4 r2 = g_ld<u32x4>(blk >= b_lo + 32 ? blk - 32 : b_lo);
    u32x4 r3 = g_ld<u32x4>(blk >= b_lo + 48 ? blk - 48 : b_lo);
    for (;;) {
      block(r0, blk);
      if (blk == b_lo) break;
      r0 = g_ld<u32x4>(at_or_lo(blk));
      blk -= 16;
      block(r1, blk);
      if (blk == b_lo) break;
      r1 = g_ld<u32x4>(at_or_lo(blk));
      blk -= 16;
      block(r2, blk);
      if (blk == b_lo) break;
      r2 = g_ld<u32x4>(at_or_lo(blk));
      blk -= 16;
      block(r3, blk);
      if (blk == b_lo) break;
      r3 = g_ld<u32x4>(at_or_lo(blk));
      blk -= 16;
    }
  }
  for (uint32_t k = 0; k < E; ++k) g_st<uint8_t>(out + nb + k, ob[k]);
  nb += E;
  g_st<uint8_t>(out, (uint8_t)x);
  g_st<uint8_t>(out + 1, (uint8_t)(x >> 8));
  g_st<uint8_t>(out + 2, (uint8_t)(x >> 16));
  g_st<uint8_t>(out + 3, (uint8_t)(x >> 24));
  seg_len[s] = nb;
}

// Byte copies of a batch of ranges: bytes [0, rev_from) forward, bytes
// [rev_from, n) taken from the end of the source backward (the rANS renorm
// bytes, emitted in the reverse of decoder order).
// The forward part is copied in whole destination words: each is the
// source's bytes at any alignment, taken from the aligned source words that
// hold them (a source word is read only when it holds one of the bytes).
__global__ void __launch_bounds__(256) ref_copy_kernel(const RefCopyOp* __restrict__ ops) {
  const RefCopyOp op = ops[blockIdx.x];
  const uint32_t t = threadIdx.x;
  const uint64_t fwd = op.rev_from < op.n ? op.rev_from : op.n;
  const uint64_t head = std::min<uint64_t>(fwd, (4u - (op.dst & 3u)) & 3u);
  const uint64_t nw = (fwd - head) / 4;
  for (uint64_t i = t; i < head; i += 256) g_st<uint8_t>(op.dst + i, gbyte(op.src + i));
  for (uint64_t w = t; w < nw; w += 256) {
    const uint64_t sa = op.src + head + 4 * w, a = sa & ~3ull;
    const uint32_t sh = (uint32_t)(sa & 3u);
    const uint32_t w0 = g_ld<uint32_t>(a), w1 = sh ? g_ld<uint32_t>(a + 4) : 0u;
    g_st<uint32_t>(op.dst + head + 4 * w, __builtin_amdgcn_alignbyte(w1, w0, sh));
  }
  for (uint64_t i = head + 4 * nw + t; i < fwd; i += 256) g_st<uint8_t>(op.dst + i, gbyte(op.src + i));
  for (uint64_t i = fwd + t; i < op.n; i += 256) g_st<uint8_t>(op.dst + i, gbyte(op.src + op.n - 1 - (i - fwd)));
}

// ---- host restatements of the reference's table construction ----

// EncSymbol (rans/compress.rs:35-68) packed for ref_rans_kernel:
// {rcp, bias, cmpl | shift << 24, freq << 20}.
void rans_encsym(uint32_t start, uint32_t freq, uint32_t out[4]) {
  uint32_t rcp, bias, shift;
  if (freq < 2) {
    bias = start + kRansScale - 1;
    rcp = 0xFFFFFFFFu;
    shift = 0;
  } else {
    uint32_t sh = 0;
    while (freq > (1u << sh)) ++sh;
    rcp = (uint32_t)((((uint64_t)1 << (sh + 31)) + freq - 1) / freq);
    bias = start;
    shift = sh - 1;
  }
  out[0] = rcp;
  out[1] = bias;
  out[2] = (kRansScale - freq) | (shift << 24);  // a 24-bit multiply reads the complement alone
  out[3] = freq << 20;                            // x at or above it sheds a byte
}

void split_four(uint64_t len, uint64_t start[4], uint64_t n[4]) {
  const uint64_t q = len / 4, r = len % 4;
  uint64_t off = 0;
  for (int i = 0; i < 4; ++i) {
    start[i] = off;
    n[i] = q + (i < (int)r ? 1 : 0);
    off += n[i];
  }
}

inline void put32(std::vector<uint8_t>& v, uint32_t x) {
  for (int i = 0; i < 4; ++i) v.push_back((uint8_t)(x >> (8 * i)));
}

inline uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

}  // namespace

int64_t RefEncoder::plan(DevCtx& ctx, const std::vector<RefJob>& jobs, std::vector<uint64_t>& payload_len) {
  hipStream_t s = ctx.stream;
  jobs_ = jobs;
  const uint32_t nj = (uint32_t)jobs.size();
  payload_len.assign(nj, 0);
  info_.assign(nj, JobInfo{});
  segs_.clear();
  if (nj == 0) return kOk;
  // ---- 1. histograms, one per split_four segment (stream_frame.rs:11-62) ----
  std::vector<RefJobDev> jd;
  std::vector<uint32_t> sub0(nj, 0);
  uint64_t max_n = 0;
  for (uint32_t j = 0; j < nj; ++j) {
    if (jobs[j].codec != kCodecHuffman && jobs[j].codec != kCodecRans) return kUnsupported;
    sub0[j] = (uint32_t)jd.size();
    if (jobs[j].n == 0) continue;
    uint64_t st[4], sn[4];
    split_four(jobs[j].n, st, sn);
    for (int i = 0; i < 4; ++i) jd.push_back(RefJobDev{jobs[j].src + st[i], sn[i]});
    max_n = std::max(max_n, sn[0]);
  }
  const uint32_t nsub = (uint32_t)jd.size();
  std::vector<uint32_t> seg_hist((size_t)nsub * 256);
  if (nsub) {
    PTWM_HIP_TRY(ctx.ref_jobs.ensure(nsub * sizeof(RefJobDev)));
    PTWM_HIP_TRY(ctx.ref_hist.ensure((size_t)nsub * 256 * sizeof(uint32_t)));
    PTWM_HIP_TRY(hipMemcpyAsync(ctx.ref_jobs.ptr, jd.data(), nsub * sizeof(RefJobDev), hipMemcpyHostToDevice, s));
    PTWM_HIP_TRY(hipMemsetAsync(ctx.ref_hist.ptr, 0, (size_t)nsub * 256 * sizeof(uint32_t), s));
    uint64_t hb = (max_n / 16 + 255) / 256;
    hb = std::max<uint64_t>(1, std::min<uint64_t>(hb, 256));
    for (uint32_t j0 = 0; j0 < nsub; j0 += 65535) {
      const uint32_t cnt = std::min<uint32_t>(65535, nsub - j0);
      hipLaunchKernelGGL(ref_hist_kernel, dim3((uint32_t)hb, cnt), dim3(256), 0, s,
                         static_cast<const RefJobDev*>(ctx.ref_jobs.ptr) + j0,
                         static_cast<uint32_t*>(ctx.ref_hist.ptr) + 256ull * j0);
      PTWM_HIP_TRY(hipGetLastError());
    }
    PTWM_HIP_TRY(hipMemcpyAsync(seg_hist.data(), ctx.ref_hist.ptr, seg_hist.size() * 4, hipMemcpyDeviceToHost, s));
    PTWM_HIP_TRY(hipStreamSynchronize(s));
  }
  std::vector<uint32_t> hist((size_t)nj * 256, 0);
  for (uint32_t j = 0; j < nj; ++j)
    if (jobs[j].n)
      for (int i = 0; i < 4; ++i)
        for (int b = 0; b < 256; ++b) hist[256ull * j + b] += seg_hist[256ull * (sub0[j] + i) + b];
  // ---- 2. tables; segments ----
  huf_codes_.assign((size_t)nj * 256, 0);
  rans_tab_.assign((size_t)nj * 256 * 4, 0);
  uint64_t scratch_words = 0, rans_scratch = 0;
  for (uint32_t j = 0; j < nj; ++j) {
    JobInfo& I = info_[j];
    const uint64_t n = jobs[j].n;
    I.raw = true;
    if (n == 0) continue;
    const uint32_t* h = &hist[256ull * j];
    if (jobs[j].codec == kCodecHuffman) {
      uint8_t lengths[256];
      uint16_t rev[256];
      if (!huf_lengths_from_freqs(h, lengths) || !huf_canonical(lengths, rev)) continue;
      uint8_t w[140];
      const int wl = huf_encode_weights(lengths, w);
      if (wl < 0) continue;
      I.header.assign(w, w + wl);
      for (int sy = 0; sy < 256; ++sy) huf_codes_[256ull * j + sy] = ((uint32_t)lengths[sy] << 16) | rev[sy];
    } else {
      uint16_t f[256], cum[256];
      int max_sym = 0;
      if (!rans_normalize_freqs(h, f, cum, &max_sym)) continue;
      I.header.push_back((uint8_t)max_sym);
      for (int i = 0; i <= max_sym; ++i) {
        I.header.push_back((uint8_t)f[i]);
        I.header.push_back((uint8_t)(f[i] >> 8));
      }
      for (int sy = 0; sy < 256; ++sy) rans_encsym(cum[sy], f[sy], &rans_tab_[(256ull * j + sy) * 4]);
    }
    I.raw = false;
    uint64_t st[4], sn[4];
    split_four(n, st, sn);
    I.seg0 = (uint32_t)segs_.size();
    for (int i = 0; i < 4; ++i) {
      RefSegDev g{};
      g.src = jobs[j].src + st[i];
      g.n = sn[i];
      g.table = j;
      if (jobs[j].codec == kCodecRans) {
        g.scratch_byte = rans_scratch;
        rans_scratch = align_up(rans_scratch + 4 + 2 * sn[i] + kRansEncSlack, 16);
      }
      segs_.push_back(g);
    }
  }
  const uint32_t ns = (uint32_t)segs_.size();
  seg_len_.assign(ns, 0);
  if (ns) {
    PTWM_HIP_TRY(ctx.ref_segs.ensure(ns * sizeof(RefSegDev)));
    PTWM_HIP_TRY(ctx.ref_seglen.ensure(ns * sizeof(unsigned long long)));
    PTWM_HIP_TRY(ctx.ref_codes.ensure(huf_codes_.size() * 4));
    PTWM_HIP_TRY(ctx.ref_rans_tab.ensure(rans_tab_.size() * 4));
    PTWM_HIP_TRY(hipMemcpyAsync(ctx.ref_segs.ptr, segs_.data(), ns * sizeof(RefSegDev), hipMemcpyHostToDevice, s));
    PTWM_HIP_TRY(hipMemcpyAsync(ctx.ref_codes.ptr, huf_codes_.data(), huf_codes_.size() * 4, hipMemcpyHostToDevice, s));
    PTWM_HIP_TRY(
        hipMemcpyAsync(ctx.ref_rans_tab.ptr, rans_tab_.data(), rans_tab_.size() * 4, hipMemcpyHostToDevice, s));
    // ---- 3. Huffman bits per segment (its histogram x code lengths); rANS segments encoded ----
    std::vector<unsigned long long> bits(ns, 0);
    for (uint32_t g = 0; g < ns; ++g) {
      const uint32_t j = segs_[g].table;
      if (jobs[j].codec != kCodecHuffman) continue;
      const uint32_t* h = &seg_hist[256ull * (sub0[j] + (g - info_[j].seg0))];
      for (int b = 0; b < 256; ++b) bits[g] += (unsigned long long)h[b] * (huf_codes_[256ull * j + b] >> 16);
    }
    // the rANS kernel gets the rANS segments only (a Huffman job's rANS
    // table row is empty)
    std::vector<RefSegDev> rsegs;
    std::vector<uint32_t> ridx;
    for (uint32_t g = 0; g < ns; ++g)
      if (jobs[segs_[g].table].codec == kCodecRans) {
        rsegs.push_back(segs_[g]);
        ridx.push_back(g);
      }
    const uint32_t nr = (uint32_t)rsegs.size();
    std::vector<unsigned long long> rlen(nr, 0);
    if (nr) {
      PTWM_HIP_TRY(ctx.ref_rans_scratch.ensure(rans_scratch));
      PTWM_HIP_TRY(ctx.ref_rans_segs.ensure(nr * sizeof(RefSegDev)));
      PTWM_HIP_TRY(ctx.ref_rans_len.ensure(nr * sizeof(unsigned long long)));
      PTWM_HIP_TRY(
          hipMemcpyAsync(ctx.ref_rans_segs.ptr, rsegs.data(), nr * sizeof(RefSegDev), hipMemcpyHostToDevice, s));
      hipLaunchKernelGGL(ref_rans_kernel, dim3((nr + kRansEncLanes - 1) / kRansEncLanes), dim3(kRansEncLanes), 0, s,
                         static_cast<const RefSegDev*>(ctx.ref_rans_segs.ptr), nr,
                         static_cast<const uint4*>(ctx.ref_rans_tab.ptr),
                         static_cast<uint8_t*>(ctx.ref_rans_scratch.ptr),
                         static_cast<unsigned long long*>(ctx.ref_rans_len.ptr));
      PTWM_HIP_TRY(hipGetLastError());
      PTWM_HIP_TRY(hipMemcpyAsync(rlen.data(), ctx.ref_rans_len.ptr, nr * 8, hipMemcpyDeviceToHost, s));
    }
    PTWM_HIP_TRY(hipStreamSynchronize(s));
    std::vector<unsigned long long> rlen_of(ns, 0);
    for (uint32_t k = 0; k < nr; ++k) {
      if (rlen[k] < 4) return kInternal;  // every rANS stream holds at least x_final
      rlen_of[ridx[k]] = rlen[k];
    }
    for (uint32_t g = 0; g < ns; ++g) {
      const RefJob& J = jobs[segs_[g].table];
      if (J.codec == kCodecHuffman) {
        seg_len_[g] = (bits[g] + 7) / 8;
        segs_[g].words = (bits[g] + 31) / 32;
        segs_[g].scratch_word = scratch_words;
        scratch_words += segs_[g].words + 1;
      } else {
        seg_len_[g] = rlen_of[g];
      }
    }
  }
  pack_words_ = scratch_words;
  // ---- 4. sizes and coded-or-raw (codecs/huffman.rs:50-87, codecs/rans.rs:50-94) ----
  for (uint32_t j = 0; j < nj; ++j) {
    JobInfo& I = info_[j];
    const uint64_t n = jobs[j].n;
    if (n == 0) {
      payload_len[j] = 1;  // [00]
      continue;
    }
    if (!I.raw) {
      uint64_t blob = I.header.size() + 16;
      for (int i = 0; i < 4; ++i) blob += seg_len_[I.seg0 + i];
      bool coded = blob < n && n <= 0xFFFFFFFFull;  // NotBeneficial when blob >= len (compress.rs:72-75)
      for (int i = 0; i < 4; ++i) coded = coded && seg_len_[I.seg0 + i] <= 0xFFFFFFFFull;
      // length_prefix::accepted (codecs/length_prefix.rs:15-56), rANS only
      if (coded && jobs[j].codec == kCodecRans) coded = n <= (1ull << 30) || n <= blob * 64;
      if (coded) {
        I.blob = blob;
        payload_len[j] = 5 + blob;
        continue;
      }
      I.raw = true;
    }
    payload_len[j] = 1 + n;  // [00] + plane
  }
  return kOk;
}

int64_t RefEncoder::write(DevCtx& ctx, const std::vector<uint64_t>& dst,
                          const std::vector<std::pair<uint64_t, std::vector<uint8_t>>>& literal,
                          const std::vector<RefCopyOp>& copies) {
  hipStream_t s = ctx.stream;
  const uint32_t nj = (uint32_t)jobs_.size();
  if (dst.size() != nj) return kInternal;
  // headers: [tag][orig_len][table header][jump table] per coded job, [00] per raw job
  std::vector<uint8_t> hdr;
  std::vector<uint64_t> hdr_off(nj + 1, 0);
  for (uint32_t j = 0; j < nj; ++j) {
    const JobInfo& I = info_[j];
    hdr_off[j] = hdr.size();
    if (I.raw) {
      hdr.push_back(0);
      continue;
    }
    hdr.push_back(1);
    put32(hdr, (uint32_t)jobs_[j].n);
    hdr.insert(hdr.end(), I.header.begin(), I.header.end());
    for (int i = 0; i < 4; ++i) put32(hdr, (uint32_t)seg_len_[I.seg0 + i]);
  }
  hdr_off[nj] = hdr.size();
  std::vector<uint64_t> lit_off;
  for (const auto& l : literal) {
    lit_off.push_back(hdr.size());
    hdr.insert(hdr.end(), l.second.begin(), l.second.end());
  }
  PTWM_HIP_TRY(ctx.ref_hdr.ensure(hdr.size() + 16));
  if (!hdr.empty()) PTWM_HIP_TRY(hipMemcpyAsync(ctx.ref_hdr.ptr, hdr.data(), hdr.size(), hipMemcpyHostToDevice, s));
  // Huffman segments packed into zeroed word scratch
  if (pack_words_) {
    PTWM_HIP_TRY(ctx.ref_pack.ensure(pack_words_ * 4));
    PTWM_HIP_TRY(hipMemsetAsync(ctx.ref_pack.ptr, 0, pack_words_ * 4, s));
    std::vector<RefSegDev> hs;
    std::vector<RefSliceDev> sl;
    std::vector<uint32_t> first;
    for (const RefSegDev& g : segs_) {
      if (jobs_[g.table].codec != kCodecHuffman || info_[g.table].raw || !g.n) continue;
      first.push_back((uint32_t)sl.size());
      for (uint64_t a = 0; a < g.n; a += kSliceSyms)
        sl.push_back(RefSliceDev{a, std::min<uint64_t>(kSliceSyms, g.n - a), (uint32_t)hs.size(), {0, 0, 0}});
      hs.push_back(g);
    }
    first.push_back((uint32_t)sl.size());
    if (!hs.empty()) {
      if (sl.size() > 0x7FFFFFFFull) return kInternal;
      const size_t b_seg = hs.size() * sizeof(RefSegDev), b_sl = sl.size() * sizeof(RefSliceDev);
      PTWM_HIP_TRY(ctx.ref_segs.ensure(b_seg + b_sl + first.size() * 4));
      PTWM_HIP_TRY(ctx.ref_seglen.ensure(sl.size() * sizeof(unsigned long long)));
      uint8_t* d = static_cast<uint8_t*>(ctx.ref_segs.ptr);
      PTWM_HIP_TRY(hipMemcpyAsync(d, hs.data(), b_seg, hipMemcpyHostToDevice, s));
      PTWM_HIP_TRY(hipMemcpyAsync(d + b_seg, sl.data(), b_sl, hipMemcpyHostToDevice, s));
      PTWM_HIP_TRY(hipMemcpyAsync(d + b_seg + b_sl, first.data(), first.size() * 4, hipMemcpyHostToDevice, s));
      const RefSegDev* d_seg = reinterpret_cast<const RefSegDev*>(d);
      const RefSliceDev* d_sl = reinterpret_cast<const RefSliceDev*>(d + b_seg);
      const uint32_t* d_first = reinterpret_cast<const uint32_t*>(d + b_seg + b_sl);
      unsigned long long* d_bits = static_cast<unsigned long long*>(ctx.ref_seglen.ptr);
      const uint32_t* d_codes = static_cast<const uint32_t*>(ctx.ref_codes.ptr);
      hipLaunchKernelGGL(ref_huf_slice_bits_kernel, dim3((uint32_t)sl.size()), dim3(256), 0, s, d_seg, d_sl, d_codes,
                         d_bits);
      hipLaunchKernelGGL(ref_huf_slice_scan_kernel, dim3((uint32_t)hs.size()), dim3(256), 0, s, d_first, d_bits);
      hipLaunchKernelGGL(ref_huf_pack_kernel, dim3((uint32_t)sl.size()), dim3(256), 0, s, d_seg, d_sl,
                         static_cast<const unsigned long long*>(d_bits), d_codes,
                         static_cast<uint32_t*>(ctx.ref_pack.ptr));
      PTWM_HIP_TRY(hipGetLastError());
    }
  }
  // gather: headers, streams, raw planes
  std::vector<RefCopyOp> ops;
  const uint64_t hdr_dev = reinterpret_cast<uint64_t>(ctx.ref_hdr.ptr);
  for (size_t k = 0; k < literal.size(); ++k)
    if (!literal[k].second.empty())
      ops.push_back(RefCopyOp{hdr_dev + lit_off[k], literal[k].first, literal[k].second.size(), ~0ull});
  // forward copies in pieces of at most kPiece bytes, one workgroup each
  constexpr uint64_t kPiece = 64ull << 10;
  const auto forward = [&](uint64_t src, uint64_t dst_addr, uint64_t n) {
    for (uint64_t o = 0; o < n; o += kPiece)
      ops.push_back(RefCopyOp{src + o, dst_addr + o, std::min<uint64_t>(kPiece, n - o), ~0ull});
  };
  for (const RefCopyOp& c : copies) forward(c.src, c.dst, c.n);
  for (uint32_t j = 0; j < nj; ++j) {
    const JobInfo& I = info_[j];
    const uint64_t hl = hdr_off[j + 1] - hdr_off[j];
    ops.push_back(RefCopyOp{hdr_dev + hdr_off[j], dst[j], hl, ~0ull});
    if (I.raw) {
      forward(jobs_[j].src, dst[j] + 1, jobs_[j].n);
      continue;
    }
    uint64_t o = dst[j] + hl;
    for (int i = 0; i < 4; ++i) {
      const RefSegDev& g = segs_[I.seg0 + i];
      const uint64_t m = seg_len_[I.seg0 + i];
      if (m) {
        if (jobs_[j].codec == kCodecHuffman) {
          // the stream is the last m bytes of the segment's word area
          const uint64_t area = reinterpret_cast<uint64_t>(ctx.ref_pack.ptr) + 4 * g.scratch_word;
          forward(area + 4 * g.words - m, o, m);
        } else {
          const uint64_t area = reinterpret_cast<uint64_t>(ctx.ref_rans_scratch.ptr) + g.scratch_byte;
          ops.push_back(RefCopyOp{area, o, m, 4});
        }
      }
      o += m;
    }
  }
  if (!ops.empty()) {
    PTWM_HIP_TRY(ctx.ref_ops.ensure(ops.size() * sizeof(RefCopyOp)));
    PTWM_HIP_TRY(hipMemcpyAsync(ctx.ref_ops.ptr, ops.data(), ops.size() * sizeof(RefCopyOp), hipMemcpyHostToDevice, s));
    for (size_t k0 = 0; k0 < ops.size(); k0 += 65535) {
      const uint32_t cnt = (uint32_t)std::min<size_t>(65535, ops.size() - k0);
      hipLaunchKernelGGL(ref_copy_kernel, dim3(cnt), dim3(256), 0, s,
                         static_cast<const RefCopyOp*>(ctx.ref_ops.ptr) + k0);
      PTWM_HIP_TRY(hipGetLastError());
    }
  }
  PTWM_HIP_TRY(hipStreamSynchronize(s));
  return kOk;
}

}  // namespace ptwm
