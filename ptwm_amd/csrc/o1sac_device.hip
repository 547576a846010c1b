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
//   sums, one 512-byte row per context, with a context -> row map.
// - Per symbol each lane holds four consecutive cumulative sums of the
//   current row (one 8-byte LDS read); four ballots of "sum <= target"
//   count the sums at or below the target, which gives the symbol of
//   binary_search_cumsum (:474-486) since the sums increase strictly, and
//   two lane reads give its interval.
// - Payload bytes and decoded symbols are staged through LDS in 4 KiB
//   pieces by the whole wavefront.
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
// LDS: [cum: 257 rows x 256 u16][row map: 256 u16][payload stage][symbol stage]
constexpr size_t kO1CumBytes = 257ull * kO1Alpha * 2;
constexpr size_t kO1Lds = kO1CumBytes + 2 * kO1Alpha + 2 * kO1Stage;

// log2(4096 / p) for p = 1..4095, the bits per symbol of max_decodable_len
// (:449-472), computed on the host with the C library's log2 (the one the
// reference's f64::log2 calls on Linux) and copied here once per device, so
// that the capacity bound's floating-point value, hence the accept / reject
// decision at its edge, is the reference's bit for bit; the division and
// floor after it are exactly rounded on both sides.
__constant__ double o1_bits[kO1Total];

__device__ __forceinline__ uint32_t ld8(const uint8_t* p) { return g_ld<uint8_t>(reinterpret_cast<uint64_t>(p)); }

__device__ __forceinline__ uint32_t wave_excl_scan(uint32_t v, uint32_t lane, uint32_t& total) {
  uint32_t incl = v;
#pragma unroll
  for (uint32_t d = 1; d < 64; d <<= 1) {
    const uint32_t u = __shfl_up(incl, d, 64);
    if (lane >= d) incl += u;
  }
  total = __shfl(incl, 63, 64);
  return incl - v;
}

__device__ __forceinline__ uint32_t wave_max(uint32_t v) {
#pragma unroll
  for (uint32_t d = 32; d >= 1; d >>= 1) v = max(v, (uint32_t)__shfl_xor(v, d, 64));
  return v;
}

// the wavefront stages payload bytes [base, base + kO1Stage) (zero past len)
__device__ void stage_payload(const uint8_t* pay, uint64_t len, uint64_t base, uint8_t* buf, uint32_t lane) {
  for (uint32_t i = lane; i < kO1Stage; i += 64) buf[i] = base + i < len ? (uint8_t)ld8(pay + base + i) : 0;
  __syncthreads();
}

}  // namespace

__global__ void __launch_bounds__(64) o1sac_decode_kernel(const DecodeJob* __restrict__ jobs,
                                                          uint32_t* __restrict__ status) {
  extern __shared__ __align__(16) uint8_t lds[];
  const DecodeJob job = jobs[blockIdx.x];
  if (job.codec != kCodecO1sac) return;
  uint16_t* const cum = reinterpret_cast<uint16_t*>(lds);
  uint16_t* const rowmap = reinterpret_cast<uint16_t*>(lds + kO1CumBytes);
  uint8_t* const inbuf = lds + kO1CumBytes + 2 * kO1Alpha;
  uint8_t* const outbuf = inbuf + kO1Stage;
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
      // context -> row: row 0 the marginal, present context c row 1 + rank(c)
      uint32_t present[4], cnt = 0;
#pragma unroll
      for (uint32_t k = 0; k < 4; ++k) {
        const uint32_t c = 4 * lane + k;
        present[k] = (ld8(state + (c >> 3)) >> (c & 7)) & 1u;
        cnt += present[k];
      }
      uint32_t t2;
      uint32_t rank = wave_excl_scan(cnt, lane, t2);
#pragma unroll
      for (uint32_t k = 0; k < 4; ++k) {
        rowmap[4 * lane + k] = present[k] ? (uint16_t)(1 + rank) : (uint16_t)0;
        rank += present[k];
      }
    }
  }
  uint32_t pmax = 0;
  if (ok) {
    bool bad = false;
    for (uint32_t r = 0; r <= pop; ++r) {
      const uint8_t* pm = state + 32 + 512ull * r;  // row 0: the marginal at 32, rows follow it
      uint32_t c[4], s = 0;
#pragma unroll
      for (uint32_t k = 0; k < 4; ++k) {
        const uint32_t i = 4 * lane + k;
        c[k] = ld8(pm + 2 * i) | (ld8(pm + 2 * i + 1) << 8);
        bad |= c[k] == 0;
        pmax = max(pmax, c[k]);
        s += c[k];
      }
      uint32_t total;
      uint32_t acc = wave_excl_scan(s, lane, total);
      bad |= total != kO1Total;
#pragma unroll
      for (uint32_t k = 0; k < 4; ++k) {
        cum[256 * r + 4 * lane + k] = (uint16_t)acc;
        acc += c[k];
      }
    }
    ok = __ballot(bad) == 0;
    pmax = wave_max(pmax);
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
  // RangeDecoder::new: five bytes preloaded; the low 32 bits of the code
  // register are all the decode reads
  uint64_t base = 0;
  stage_payload(pay, plen, 0, inbuf, lane);
  uint32_t code = ((uint32_t)inbuf[1] << 24) | ((uint32_t)inbuf[2] << 16) | ((uint32_t)inbuf[3] << 8) | inbuf[4];
  uint64_t pos = 5;
  uint32_t low = 0, range = 0xFFFFFFFFu, prev = 0;
  uint64_t row_pos = 0;
  uint8_t* dst = reinterpret_cast<uint8_t*>(job.dst);
  for (uint64_t i = 0; i < n; ++i) {
    const uint32_t row = row_pos == 0 ? 0u : rowmap[prev];
    const uint32_t rpt = range >> 12;  // range / 4096
    uint32_t target = (code - low) / rpt;
    target = target > kO1Total - 1 ? kO1Total - 1 : target;
    const uint2 q = *reinterpret_cast<const uint2*>(cum + 256 * row + 4 * lane);
    const uint32_t c0 = q.x & 0xFFFFu, c1 = q.x >> 16, c2 = q.y & 0xFFFFu, c3 = q.y >> 16;
    const uint32_t cnt = __popcll(__ballot(c0 <= target)) + __popcll(__ballot(c1 <= target)) +
                         __popcll(__ballot(c2 <= target)) + __popcll(__ballot(c3 <= target));
    const uint32_t sym = cnt - 1;  // cum[0] = 0 <= target: cnt >= 1
    const uint32_t k0 = sym & 3u, k1 = (sym + 1) & 3u;
    const uint32_t lo = __builtin_amdgcn_readlane(k0 == 0 ? c0 : k0 == 1 ? c1 : k0 == 2 ? c2 : c3, sym >> 2);
    const uint32_t hi = sym == 255 ? kO1Total
                                   : __builtin_amdgcn_readlane(k1 == 0 ? c0 : k1 == 1 ? c1 : k1 == 2 ? c2 : c3,
                                                               (sym + 1) >> 2);
    low += lo * rpt;  // RangeDecoder::advance; low stays masked to 32 bits
    range = (hi - lo) * rpt;
    while (range < (1u << 24)) {
      if (pos - base == kO1Stage) {
        base += kO1Stage;
        __syncthreads();
        stage_payload(pay, plen, base, inbuf, lane);
      }
      code = (code << 8) | inbuf[pos - base];
      ++pos;
      low = (low & 0xFFFFFFu) << 8;
      range <<= 8;
    }
    if (lane == 0) outbuf[i % kO1Stage] = (uint8_t)sym;
    prev = sym;
    row_pos = row_pos + 1 == rl ? 0 : row_pos + 1;
    if ((i + 1) % kO1Stage == 0 || i + 1 == n) {
      __syncthreads();
      const uint64_t o = i / kO1Stage * kO1Stage, m = i + 1 - o;
      for (uint32_t j = lane; j < m; j += 64) g_st<uint8_t>(reinterpret_cast<uint64_t>(dst + o + j), outbuf[j]);
      __syncthreads();
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
