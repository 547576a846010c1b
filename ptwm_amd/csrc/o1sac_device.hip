// o1sac_device.hip -- Order1ScaleAC (codec 0x0011) payloads on the device.
//
// Order1ScaleAC codes a scale plane with a 32-bit carry-propagating range
// coder under per-context PMFs: the first symbol of each row under the
// marginal PMF, every other one under the PMF of its predecessor's context
// when the state holds one (codecs/order1_scale_ac.rs:593-707,
// range_coder.rs:14-197).  One coder state runs through the whole payload,
// so a payload is one serial chain by its definition: one wavefront per
// payload (or chunk frame), every lane holding the same coder state.
//
// - The state ([bitmap 32 B][marginal u16 x 256][present rows u16 x 256])
//   is checked as deserialize_state checks it (:159-203: length, no zero
//   count, every PMF summing to 4096) and laid out in LDS as cumulative
//   sums, one 520-byte row per context (a context without a row of its own
//   holds a copy of the marginal) and one for the marginal, each row's 256
//   sums followed by 4096, so the row of the next symbol is an address
//   computed from the symbol, with no table between them.
// - Per symbol each lane holds four consecutive cumulative sums c of the
//   row and the next one.  binary_search_cumsum (:474-486) looks for the
//   last sum c <= min(offset / rpt, 4095); every sum of symbols 0..255 is at
//   most 4095, so that is the last c with c * rpt <= offset, and no division
//   is needed.  Four ballots of that test count the symbol; each lane picks
//   its own last product under the offset and the one after it, and two
//   lane reads at the last lane whose first test holds give lo * rpt and
//   hi * rpt.
// - The coder state is wave-uniform; renormalisation shifts by clz(range)
//   rounded down to whole bytes, taken from a 64-bit register window of
//   payload bytes refilled a word at a time from the LDS stage (the word
//   is read one refill ahead).  Payload bytes are staged through LDS in
//   4 KiB pieces; decoded symbols collect one per lane and are stored 64 at
//   a time.
#include <hip/hip_runtime.h>

#include <cmath>
#include <mutex>

#include "decode_sync.h"

namespace ptwm {

namespace {

constexpr uint32_t kO1Alpha = 256;
constexpr uint32_t kO1Total = 4096;  // quantize.rs:8 ORDER1_QUANT_TOTAL
constexpr uint32_t kO1Hdr = 32 + 2 * kO1Alpha;
constexpr uint32_t kO1Stage = 4096;
// LDS: [rows: 257 x (256 cumulative sums + 4096) at a 520-byte stride]
// [payload stage]; row c (0..255) serves the symbol after symbol c, row 256
// (the marginal) a row's first symbol
constexpr uint32_t kO1RowBytes = 520;
constexpr uint32_t kO1Marginal = 256;
constexpr size_t kO1CumBytes = 257ull * kO1RowBytes;
constexpr size_t kO1Lds = kO1CumBytes + kO1Stage;

// log2(4096 / p) for p = 1..4095, the bits per symbol of max_decodable_len
// (:449-472), computed on the host with the C library's log2 (the one the
// reference's f64::log2 calls on Linux) and copied here once per device, so
// that the capacity bound's floating-point value, hence the accept / reject
// decision at its edge, is the reference's bit for bit; the division and
// floor after it are exactly rounded on both sides.
__constant__ double o1_bits[kO1Total];

__device__ __forceinline__ uint32_t ld8(const uint8_t* p) { return g_ld<uint8_t>(reinterpret_cast<uint64_t>(p)); }

// exclusive prefix sum over the wavefront (total: the sum of all lanes):
// an inclusive scan within each row of 16 lanes by row shifts, then each
// row's predecessors' totals through the row broadcasts of lanes 15 and 31
__device__ __forceinline__ uint32_t wave_excl_scan(uint32_t v, uint32_t lane, uint32_t& total) {
  (void)lane;
  uint32_t x = v;
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xF, 0xF, false);  // row_shr:2
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xF, 0xF, false);  // row_shr:4
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xF, 0xF, false);  // row_shr:8
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xA, 0xF, false);  // row_bcast:15 -> rows 1, 3
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xC, 0xF, false);  // row_bcast:31 -> rows 2, 3
  total = __builtin_amdgcn_readlane(x, 63);
  return x - v;
}

__device__ __forceinline__ uint32_t wave_max(uint32_t v) {
#pragma unroll
  for (uint32_t d = 32; d >= 1; d >>= 1) v = max(v, (uint32_t)__shfl_xor(v, d, 64));
  return v;
}

// the wavefront stages payload bytes [base, base + kO1Stage) (zero past len)
// as words: each lane's sixteen words are loaded byte by byte from clamped
// addresses, all loads issued before the first word is written
__device__ void stage_payload(const uint8_t* pay, uint64_t len, uint64_t base, uint8_t* buf, uint32_t lane) {
  uint32_t w[16];
  if (len == 0) {
#pragma unroll
    for (uint32_t k = 0; k < 16; ++k) w[k] = 0;
  } else {
#pragma unroll
    for (uint32_t k = 0; k < 16; ++k) {
      const uint64_t a = base + 4ull * (64 * k + lane);
      uint32_t v = 0;
#pragma unroll
      for (uint32_t b = 0; b < 4; ++b) {
        const uint32_t x = ld8(pay + (a + b < len ? a + b : len - 1));
        v |= (a + b < len ? x : 0u) << (8 * b);
      }
      w[k] = v;
    }
  }
#pragma unroll
  for (uint32_t k = 0; k < 16; ++k) reinterpret_cast<uint32_t*>(buf)[64 * k + lane] = w[k];
  __syncthreads();
}

// a payload word read from the LDS stage at byte offset o (a multiple of 4)
__device__ __forceinline__ uint32_t stage_word(const uint8_t* buf, uint32_t o) {
  return *reinterpret_cast<const uint32_t*>(buf + o);
}

// a staged word, most significant byte first, wave-uniform
__device__ __forceinline__ uint32_t word_be(uint32_t w) { return __builtin_amdgcn_readfirstlane(__builtin_bswap32(w)); }

}  // namespace

__global__ void __launch_bounds__(64) o1sac_decode_kernel(const DecodeJob* __restrict__ jobs,
                                                          uint32_t* __restrict__ status) {
  extern __shared__ __align__(16) uint8_t lds[];
  const DecodeJob job = jobs[blockIdx.x];
  if (job.codec != kCodecO1sac) return;
  uint8_t* const inbuf = lds + kO1CumBytes;
  const uint32_t lane = threadIdx.x;
  const uint8_t* src = reinterpret_cast<const uint8_t*>(job.src);
  const uint64_t n = job.dst_len;
  // the state and the payload: a chunk frame [ver][state_len u32][state]
  // [payload] (container.rs:2010-2049), else the plan's state bytes
  const uint8_t* state;
  uint64_t state_len, plen;
  uint32_t version;
  const uint8_t* pay;
  if (job.framed) {
    if (job.src_len < 5) {
      if (lane == 0) status[blockIdx.x] = kStBadFrame;
      return;
    }
    state_len = ld8(src + 1) | (ld8(src + 2) << 8) | (ld8(src + 3) << 16) | ((uint64_t)ld8(src + 4) << 24);
    if (job.src_len - 5 < state_len) {
      if (lane == 0) status[blockIdx.x] = kStBadFrame;
      return;
    }
    version = ld8(src);
    state = src + 5;
    pay = src + 5 + state_len;
    plen = job.src_len - 5 - state_len;
  } else {
    state = reinterpret_cast<const uint8_t*>((uint64_t)job.pad[0] | ((uint64_t)job.pad[1] << 32));
    state_len = job.pad[2] & 0xFFFFFFu;
    version = job.pad[2] >> 24;
    pay = src;
    plen = job.src_len;
  }
  const uint32_t row_len_plan = job.pad[3];
  // decode(): the state version (order1_scale_ac.rs:648-657), then
  // deserialize_state's checks
  uint32_t pop = 0;
  bool ok = version == 1 && state_len >= kO1Hdr;
  if (ok) {
    const uint32_t b = lane < 32 ? ld8(state + lane) : 0u;
    pop = __popc(b);
    uint32_t total;
    (void)wave_excl_scan(pop, lane, total);
    pop = total;
    ok = state_len == (uint64_t)kO1Hdr + (uint64_t)pop * 2 * kO1Alpha;
    if (ok) {
      // present context c has state row 1 + rank(c) (row 0 is the
      // marginal); ctx_of[r] = the context of state row r, staged in the
      // payload buffer until the rows are built
      uint32_t present[4], cnt = 0;
#pragma unroll
      for (uint32_t k = 0; k < 4; ++k) {
        const uint32_t c = 4 * lane + k;
        present[k] = (ld8(state + (c >> 3)) >> (c & 7)) & 1u;
        cnt += present[k];
      }
      uint32_t t2;
      uint32_t rank = wave_excl_scan(cnt, lane, t2);
      uint16_t* const ctx_of = reinterpret_cast<uint16_t*>(inbuf);
      if (lane == 0) ctx_of[0] = (uint16_t)kO1Marginal;
#pragma unroll
      for (uint32_t k = 0; k < 4; ++k) {
        if (present[k]) ctx_of[1 + rank] = (uint16_t)(4 * lane + k);
        rank += present[k];
      }
    }
  }
  uint32_t pmax = 0;
  if (ok) {
    __syncthreads();
    const uint16_t* const ctx_of = reinterpret_cast<const uint16_t*>(inbuf);
    bool bad = false;
    // each state row's counts are loaded while the previous one is summed
    uint32_t nc[4];
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) nc[k] = ld8(state + 32 + 8 * lane + 2 * k) | (ld8(state + 33 + 8 * lane + 2 * k) << 8);
    for (uint32_t r = 0; r <= pop; ++r) {
      uint32_t c[4], s = 0;
#pragma unroll
      for (uint32_t k = 0; k < 4; ++k) c[k] = nc[k];
      if (r < pop) {
        const uint8_t* pm = state + 32 + 512ull * (r + 1);  // rows follow the marginal at 32
#pragma unroll
        for (uint32_t k = 0; k < 4; ++k) nc[k] = ld8(pm + 8 * lane + 2 * k) | (ld8(pm + 8 * lane + 2 * k + 1) << 8);
      }
#pragma unroll
      for (uint32_t k = 0; k < 4; ++k) {
        bad |= c[k] == 0;
        pmax = max(pmax, c[k]);
        s += c[k];
      }
      uint32_t total;
      const uint32_t acc = wave_excl_scan(s, lane, total);
      bad |= total != kO1Total;
      uint8_t* const row = lds + (size_t)ctx_of[r] * kO1RowBytes;
      const uint32_t a1 = acc + c[0], a2 = a1 + c[1], a3 = a2 + c[2];
      *reinterpret_cast<uint2*>(row + 8 * lane) = make_uint2((acc & 0xFFFFu) | (a1 << 16), (a2 & 0xFFFFu) | (a3 << 16));
      if (lane == 0) *reinterpret_cast<uint16_t*>(row + 512) = (uint16_t)kO1Total;
    }
    ok = __ballot(bad) == 0;
    pmax = wave_max(pmax);
    if (ok) {
      // contexts with no row of their own take the marginal's
      __syncthreads();
      const uint2 mq = *reinterpret_cast<const uint2*>(lds + kO1Marginal * kO1RowBytes + 8 * lane);
      const uint32_t bm = lane < 32 ? ld8(state + lane) : 0u;
      for (uint32_t c = 0; c < kO1Alpha; ++c) {
        if ((__builtin_amdgcn_readlane(bm, c >> 3) >> (c & 7)) & 1u) continue;
        uint8_t* const row = lds + (size_t)c * kO1RowBytes;
        *reinterpret_cast<uint2*>(row + 8 * lane) = mq;
        if (lane == 0) *reinterpret_cast<uint16_t*>(row + 512) = (uint16_t)kO1Total;
      }
    }
  }
  if (!ok) {
    if (lane == 0) status[blockIdx.x] = kStBadHeader;
    return;
  }
  // row length (:411-432) and the payload's capacity bound (:449-472)
  const uint64_t rl = row_len_plan ? row_len_plan : (n ? n : 1);
  bool len_ok = n % rl == 0;
  if (len_ok && pmax < kO1Total) {
    const double bits = o1_bits[pmax];
    const double budget = 8.0 * (double)(plen > 5 ? plen - 5 : 0);
    const double cap = floor(budget / bits) + 1.0;
    len_ok = cap >= 18446744073709551615.0 || (double)n <= cap;
  }
  if (!len_ok) {
    if (lane == 0) status[blockIdx.x] = kStBadLength;
    return;
  }
  __syncthreads();
  // RangeDecoder::new: five bytes preloaded (the first, the encoder's
  // alignment byte, leaves the low 32 bits of the code register, which are
  // all the decode reads); bytes 5..7 start the window, word 8 is next
  uint64_t sbase = 0;
  stage_payload(pay, plen, 0, inbuf, lane);
  const uint32_t w0 = word_be(stage_word(inbuf, 0)), w1 = word_be(stage_word(inbuf, 4));
  uint32_t code = (w0 << 8) | (w1 >> 24);
  uint64_t win = (uint64_t)(w1 << 8) << 32;  // payload bytes, first in the top byte
  uint32_t avail = 3;                         // bytes held in win
  uint64_t fetch = 8;                         // payload offset of the next word
  uint32_t next = stage_word(inbuf, 8);  // read here, used a refill later
  uint32_t low = 0, range = 0xFFFFFFFFu;
  uint8_t* const dst = reinterpret_cast<uint8_t*>(job.dst);
  const uint8_t* const lrow = lds + 8 * lane;
  uint64_t i = 0, row_pos = 0;
  uint32_t wpos = 0, outv = 0;  // symbols i - wpos .. i - 1, one per lane
  uint32_t sym = 0;
  while (i < n) {
    // this lane's sums of the row of the segment's first symbol (a row's
    // first symbol: the marginal); each step then reads the next symbol's
    // row as soon as its own symbol is known
    const uint8_t* rp = lrow + (row_pos == 0 ? kO1Marginal : sym) * kO1RowBytes;
    uint2 q = *reinterpret_cast<const uint2*>(rp);
    uint32_t c4 = *reinterpret_cast<const uint16_t*>(rp + 8);
    uint64_t seg = n - i;
    if (rl - row_pos < seg) seg = rl - row_pos;
    if (64 - wpos < seg) seg = 64 - wpos;
    const uint32_t end = wpos + (uint32_t)seg;
    for (; wpos < end; ++wpos) {
      const uint32_t rpt = range >> 12;  // range / 4096
      const uint32_t off = code - low;   // (code - low) mod 2^32
      // c * rpt < 2^32 for c <= 4096, rpt < 2^20
      const uint32_t p0 = __umul24(q.x & 0xFFFFu, rpt), p1 = __umul24(q.x >> 16, rpt);
      const uint32_t p2 = __umul24(q.y & 0xFFFFu, rpt), p3 = __umul24(q.y >> 16, rpt);
      const uint32_t p4 = __umul24(c4, rpt);
      const bool t0 = p0 <= off, t1 = p1 <= off, t2 = p2 <= off, t3 = p3 <= off;
      const uint64_t m0 = __ballot(t0);
      sym = __popcll(m0) + __popcll(__ballot(t1)) + __popcll(__ballot(t2)) +
                           __popcll(__ballot(t3)) - 1;  // lane 0's first sum is 0: m0 != 0
      const uint32_t at = __popcll(m0) - 1;           // the lane holding the symbol's sum
      const uint32_t lo_v = t3 ? p3 : t2 ? p2 : t1 ? p1 : p0;
      const uint32_t hi_v = t3 ? p4 : t2 ? p3 : t1 ? p2 : p1;
      // the next step's row (read past a segment's end is unused)
      rp = lrow + sym * kO1RowBytes;
      q = *reinterpret_cast<const uint2*>(rp);
      c4 = *reinterpret_cast<const uint16_t*>(rp + 8);
      const uint32_t lo = __builtin_amdgcn_readlane(lo_v, at), hi = __builtin_amdgcn_readlane(hi_v, at);
      low += lo;  // RangeDecoder::advance; low stays masked to 32 bits
      range = hi - lo;
      // renormalise: whole bytes until range >= 2^24 (range >= 2^12, so at
      // most two); low and code shift in 32 bits
      const uint32_t sh = __builtin_clz(range) & ~7u;
      code = (uint32_t)(((((uint64_t)code << 32) | (win >> 32)) << sh) >> 32);
      win <<= sh;
      low <<= sh;
      range <<= sh;
      avail -= sh >> 3;
      if (avail < 4) {
        win |= (uint64_t)word_be(next) << (32 - 8 * avail);
        avail += 4;
        fetch += 4;
        if (fetch - sbase == kO1Stage) {
          sbase += kO1Stage;
          __syncthreads();
          stage_payload(pay, plen, sbase, inbuf, lane);
        }
        next = stage_word(inbuf, (uint32_t)(fetch - sbase));
      }
      outv = lane == wpos ? sym : outv;
    }
    i += seg;
    row_pos += seg;
    if (row_pos == rl) row_pos = 0;
    if (wpos == 64 || i == n) {
      if (lane < wpos) g_st<uint8_t>(reinterpret_cast<uint64_t>(dst + (i - wpos) + lane), (uint8_t)outv);
      wpos = 0;
    }
  }
  if (lane == 0) status[blockIdx.x] = kStOk;
}

hipError_t launch_o1sac_decode(const DecodeJob* jobs_dev, uint32_t* status_dev, uint32_t n_jobs, hipStream_t stream) {
  if (n_jobs == 0) return hipSuccess;
  static std::mutex mu;
  static bool bits_ready[64] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  {
    std::lock_guard<std::mutex> lk(mu);
    if (!bits_ready[dev]) {
      double bits[kO1Total];
      bits[0] = 0.0;  // p_max >= 1 in a checked state
      for (uint32_t p = 1; p < kO1Total; ++p) bits[p] = std::log2((double)kO1Total / (double)p);
      e = hipMemcpyToSymbol(HIP_SYMBOL(o1_bits), bits, sizeof bits);
      if (e != hipSuccess) return e;
      bits_ready[dev] = true;
    }
  }
  e = hipFuncSetAttribute((const void*)o1sac_decode_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)kO1Lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(o1sac_decode_kernel, dim3(n_jobs), dim3(64), kO1Lds, stream, jobs_dev, status_dev);
  return hipGetLastError();
}

}  // namespace ptwm
