// plane_ops.hip -- plane ops on terminal planes: their inverses for the
// decode, the ops themselves for the encoder.
//
// The reference applies these ops to one terminal plane of a split chain
// (python/ptwm/preprocessing/_chains.py:360-600: the exponent plane through
// IntDelta or PredictorXor, a mantissa plane through MantissaZeroStrip);
// the decode runs their inverses after the plane's CRC check and before the
// merge (container.rs:2152-2170, chain/dispatch.rs:96-122).
//
// - IntDelta (transforms/int_delta.rs:38-46): the inverse is the running
//   wrapping sum of the plane's elements, a prefix scan: per 4 KiB tile a
//   sum (pass 1), per plane an exclusive scan of its tile sums (pass 2), per
//   tile an in-thread / workgroup scan plus the tile's prefix (pass 3).
//   Element widths 1, 2, 4 and 8 bytes.
// - MantissaZeroStrip (transforms/mantissa_zero.rs): b << k per byte, one
//   streaming pass.
// - PredictorXor (transforms/predictor_xor.rs:10-25): every value depends
//   on the 2^16-entry table of the values before it, so a plane is one
//   serial chain by its definition.  One workgroup per plane keeps the table
//   in LDS (element widths 1 and 2: 64 KiB / 128 KiB) and streams the plane
//   through LDS in 4 KiB chunks; one lane runs the recurrence.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>

#include "plane_ops.h"

namespace ptwm {

namespace {

constexpr uint32_t kTile = 4096;      // bytes per tile: 256 threads x 16 bytes
constexpr uint32_t kPxChunk = 4096;   // PredictorXor staging chunk (bytes)
constexpr uint32_t kMaxGrid = 65536;  // workgroups per launch (tile loops beyond)

// job of launch tile t: the last j with jobs[j].tile0 <= t
__device__ uint32_t find_job(const PlaneOpJob* __restrict__ jobs, uint32_t n_jobs, uint64_t t) {
  uint32_t lo = 0, hi = n_jobs;
  while (hi - lo > 1) {
    const uint32_t mid = (lo + hi) / 2;
    if (jobs[mid].tile0 <= t) lo = mid;
    else hi = mid;
  }
  return lo;
}

// the 16 bytes at offset o (a multiple of 16) of an n-byte plane; bytes at
// or past n read as zero
__device__ __forceinline__ void load16(uint64_t base, uint64_t o, uint64_t n, uint32_t (&w)[4]) {
  if (o + 16 <= n) {
    const u32x4 v = g_ld<u32x4>(base + o);
    w[0] = v.x;
    w[1] = v.y;
    w[2] = v.z;
    w[3] = v.w;
    return;
  }
  w[0] = w[1] = w[2] = w[3] = 0;
  for (uint64_t b = o; b < n; ++b) w[(b - o) >> 2] |= (uint32_t)g_ld<uint8_t>(base + b) << (8 * ((b - o) & 3));
}

__device__ __forceinline__ void store16(uint64_t base, uint64_t o, uint64_t n, const uint32_t (&w)[4]) {
  if (o + 16 <= n) {
    g_st<u32x4>(base + o, u32x4_make(w[0], w[1], w[2], w[3]));
    return;
  }
  for (uint64_t b = o; b < n; ++b) g_st<uint8_t>(base + b, (uint8_t)(w[(b - o) >> 2] >> (8 * ((b - o) & 3))));
}

// element e (little endian, W bytes) of 16 bytes held as four words
template <uint32_t W>
__device__ __forceinline__ uint64_t get_elem(const uint32_t (&w)[4], uint32_t e) {
  if constexpr (W == 1) return (w[e >> 2] >> (8 * (e & 3))) & 0xFFu;
  else if constexpr (W == 2) return (w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
  else if constexpr (W == 4) return w[e];
  else return (uint64_t)w[2 * e] | ((uint64_t)w[2 * e + 1] << 32);
}

template <uint32_t W>
__device__ __forceinline__ void set_elem(uint32_t (&w)[4], uint32_t e, uint64_t v) {
  if constexpr (W == 1) {
    const uint32_t s = 8 * (e & 3);
    w[e >> 2] = (w[e >> 2] & ~(0xFFu << s)) | (((uint32_t)v & 0xFFu) << s);
  } else if constexpr (W == 2) {
    const uint32_t s = 16 * (e & 1);
    w[e >> 1] = (w[e >> 1] & ~(0xFFFFu << s)) | (((uint32_t)v & 0xFFFFu) << s);
  } else if constexpr (W == 4) {
    w[e] = (uint32_t)v;
  } else {
    w[2 * e] = (uint32_t)v;
    w[2 * e + 1] = (uint32_t)(v >> 32);
  }
}

// Exclusive scan of v over the 256 threads (sums wrap at 64 bits, which
// preserves every narrower width); *total = the sum of all.  sh: 4 words.
__device__ __forceinline__ uint64_t block_excl_scan(uint64_t v, uint64_t* sh, uint64_t& total) {
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  uint64_t incl = v;
#pragma unroll
  for (uint32_t d = 1; d < 64; d <<= 1) {
    const uint64_t u = __shfl_up(incl, d, 64);
    if (lane >= d) incl += u;
  }
  if (lane == 63) sh[wave] = incl;
  __syncthreads();
  uint64_t base = 0;
  total = 0;
#pragma unroll
  for (uint32_t k = 0; k < 4; ++k) {
    if (k < wave) base += sh[k];
    total += sh[k];
  }
  __syncthreads();  // sh is reused by the next call
  return base + incl - v;
}

// IntDelta pass 1: the sum of each tile's elements
template <uint32_t W>
__global__ void __launch_bounds__(256) idelta_sums(const PlaneOpJob* __restrict__ jobs, uint32_t n_jobs,
                                                   uint64_t n_tiles, uint64_t* __restrict__ sums) {
  __shared__ uint64_t sh[4];
  for (uint64_t t = blockIdx.x; t < n_tiles; t += gridDim.x) {
    const PlaneOpJob& J = jobs[find_job(jobs, n_jobs, t)];
    const uint64_t tile = t - J.tile0;
    const uint64_t o = tile * kTile + 16ull * threadIdx.x;
    uint32_t w[4] = {0, 0, 0, 0};
    if (o < J.n) load16(J.src, o, J.n, w);
    uint64_t s = 0;
#pragma unroll
    for (uint32_t e = 0; e < 16 / W; ++e) s += get_elem<W>(w, e);
    uint64_t total;
    (void)block_excl_scan(s, sh, total);
    if (threadIdx.x == 0) g_st<uint64_t>(reinterpret_cast<uint64_t>(sums + J.aux + tile), total);
  }
}

// IntDelta pass 2: each job's tile sums become exclusive prefixes (one
// workgroup per job)
__global__ void __launch_bounds__(256) idelta_scan_sums(const PlaneOpJob* __restrict__ jobs,
                                                        uint64_t* __restrict__ sums) {
  __shared__ uint64_t sh[4];
  const PlaneOpJob& J = jobs[blockIdx.x];
  const uint64_t nt = (J.n + kTile - 1) / kTile;
  uint64_t carry = 0;
  for (uint64_t b = 0; b < nt; b += 256) {
    const uint64_t i = b + threadIdx.x;
    const uint64_t a = reinterpret_cast<uint64_t>(sums + J.aux + i);
    const uint64_t v = i < nt ? g_ld<uint64_t>(a) : 0;
    uint64_t total;
    const uint64_t ex = block_excl_scan(v, sh, total);
    if (i < nt) g_st<uint64_t>(a, carry + ex);
    carry += total;
  }
}

// IntDelta pass 3: each element becomes the running sum of the plane up to
// and including itself (int_delta.rs delta_inverse: out[0] = in[0],
// out[i] = out[i-1] + in[i], wrapping at the width)
template <uint32_t W>
__global__ void __launch_bounds__(256) idelta_apply(const PlaneOpJob* __restrict__ jobs, uint32_t n_jobs,
                                                    uint64_t n_tiles, const uint64_t* __restrict__ sums) {
  __shared__ uint64_t sh[4];
  for (uint64_t t = blockIdx.x; t < n_tiles; t += gridDim.x) {
    const PlaneOpJob& J = jobs[find_job(jobs, n_jobs, t)];
    const uint64_t tile = t - J.tile0;
    const uint64_t o = tile * kTile + 16ull * threadIdx.x;
    uint32_t w[4] = {0, 0, 0, 0};
    if (o < J.n) load16(J.src, o, J.n, w);
    uint64_t r = 0;
#pragma unroll
    for (uint32_t e = 0; e < 16 / W; ++e) {
      r += get_elem<W>(w, e);
      set_elem<W>(w, e, r);
    }
    uint64_t total;
    const uint64_t pre = block_excl_scan(r, sh, total) + g_ld<uint64_t>(reinterpret_cast<uint64_t>(sums + J.aux + tile));
#pragma unroll
    for (uint32_t e = 0; e < 16 / W; ++e) set_elem<W>(w, e, get_elem<W>(w, e) + pre);
    if (o < J.n) store16(J.dst, o, J.n, w);
  }
}

// MantissaZeroStrip inverse: every byte b becomes (b << k) & 0xFF
__global__ void __launch_bounds__(256) mzs_inverse(const PlaneOpJob* __restrict__ jobs, uint32_t n_jobs,
                                                   uint64_t n_tiles) {
  for (uint64_t t = blockIdx.x; t < n_tiles; t += gridDim.x) {
    const PlaneOpJob& J = jobs[find_job(jobs, n_jobs, t)];
    const uint64_t o = (t - J.tile0) * kTile + 16ull * threadIdx.x;
    if (o >= J.n) continue;
    const uint32_t k = J.param;
    const uint32_t m = ((0xFFu << k) & 0xFFu) * 0x01010101u;
    uint32_t w[4];
    load16(J.src, o, J.n, w);
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = (w[i] << k) & m;
    store16(J.dst, o, J.n, w);
  }
}

// PredictorXor inverse, one wavefront per plane (jobs[which[blockIdx.x]]),
// element width W (1 or 2).  LDS: [table: 2^16 entries of W bytes]
// [residual chunk, kPxChunk bytes][value chunk, kPxChunk bytes].  The
// wavefront stages each chunk of residuals with 16-byte loads, lane 0 runs
// the recurrence of predictor_xor.rs decode_specialized (prediction =
// table[hash], value = residual ^ prediction, table[hash] = value,
// hash = ((hash << 6) ^ value) & 0xFFFF), and the wavefront stores the
// values.
template <uint32_t W, bool kForward = false>
__global__ void __launch_bounds__(64) pxor_inverse(const PlaneOpJob* __restrict__ jobs,
                                                   const uint32_t* __restrict__ which) {
  extern __shared__ __align__(16) uint32_t lds[];
  constexpr uint32_t kTabWords = (65536u * W) / 4;
  uint32_t* const in = lds + kTabWords;
  uint32_t* const outw = in + kPxChunk / 4;
  const PlaneOpJob& J = jobs[which[blockIdx.x]];
  const uint32_t lane = threadIdx.x;
  for (uint32_t i = lane; i < kTabWords; i += 64) lds[i] = 0;
  __syncthreads();
  uint32_t h = 0;
  for (uint64_t c = 0; c < J.n; c += kPxChunk) {
    const uint64_t len = J.n - c < kPxChunk ? J.n - c : kPxChunk;
    for (uint32_t q = 16 * lane; q < len; q += 1024) {
      uint32_t w[4];
      load16(J.src, c + q, J.n, w);
      *reinterpret_cast<u32x4*>(in + q / 4) = u32x4_make(w[0], w[1], w[2], w[3]);
    }
    __syncthreads();
    if (lane == 0) {
      if constexpr (W == 1) {
        uint8_t* const tab = reinterpret_cast<uint8_t*>(lds);
        for (uint32_t i = 0; i < len; i += 4) {
          const uint32_t x4 = in[i / 4];
          uint32_t o4 = 0;
#pragma unroll
          for (uint32_t k = 0; k < 4; ++k) {
            const uint32_t x = (x4 >> (8 * k)) & 0xFFu, r = x ^ tab[h];
            const uint32_t v = kForward ? x : r;  // the value the table and hash follow
            tab[h] = (uint8_t)v;
            h = ((h << 6) ^ v) & 0xFFFFu;
            o4 |= r << (8 * k);
          }
          outw[i / 4] = o4;
        }
      } else {
        uint16_t* const tab = reinterpret_cast<uint16_t*>(lds);
        for (uint32_t i = 0; i < len; i += 4) {
          const uint32_t x4 = in[i / 4];
          uint32_t o4 = 0;
#pragma unroll
          for (uint32_t k = 0; k < 2; ++k) {
            const uint32_t x = (x4 >> (16 * k)) & 0xFFFFu, r = x ^ tab[h];
            const uint32_t v = kForward ? x : r;
            tab[h] = (uint16_t)v;
            h = ((h << 6) ^ v) & 0xFFFFu;
            o4 |= r << (16 * k);
          }
          outw[i / 4] = o4;
        }
      }
    }
    __syncthreads();
    for (uint32_t q = 16 * lane; q < len; q += 1024) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(outw + q / 4);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
      store16(J.dst, c + q, J.n, w);
    }
    __syncthreads();
  }
}

// ---- forward ops (the encoder's direction) ----

// IntDelta forward (int_delta.rs:38-46): out[0] = in[0], out[i] = in[i] -
// in[i-1] at the element width; each thread also reads the element before
// its 16 bytes.
template <uint32_t W>
__global__ void __launch_bounds__(256) idelta_forward(const PlaneOpJob* __restrict__ jobs, uint32_t n_jobs,
                                                      uint64_t n_tiles) {
  for (uint64_t t = blockIdx.x; t < n_tiles; t += gridDim.x) {
    const PlaneOpJob& J = jobs[find_job(jobs, n_jobs, t)];
    const uint64_t o = (t - J.tile0) * kTile + 16ull * threadIdx.x;
    if (o >= J.n) continue;
    uint32_t w[4], v[4] = {0, 0, 0, 0};
    load16(J.src, o, J.n, w);
    uint64_t prev = 0;
    if (o >= W) {
      uint32_t pw[4];
      load16(J.src, o - 16, J.n, pw);
      prev = get_elem<W>(pw, 16 / W - 1);
    }
#pragma unroll
    for (uint32_t e = 0; e < 16 / W; ++e) {
      const uint64_t x = get_elem<W>(w, e);
      set_elem<W>(v, e, o + e * W == 0 ? x : x - prev);
      prev = x;
    }
    store16(J.dst, o, J.n, v);
  }
}

// MantissaZeroStrip forward (mantissa_zero.rs forward): b >> k; a byte with
// a nonzero low k bits refuses the plane (flag[job] = 1)
__global__ void __launch_bounds__(256) mzs_forward(const PlaneOpJob* __restrict__ jobs, uint32_t n_jobs,
                                                   uint64_t n_tiles, uint32_t* __restrict__ flag) {
  for (uint64_t t = blockIdx.x; t < n_tiles; t += gridDim.x) {
    const uint32_t j = find_job(jobs, n_jobs, t);
    const PlaneOpJob& J = jobs[j];
    const uint64_t o = (t - J.tile0) * kTile + 16ull * threadIdx.x;
    if (o >= J.n) continue;
    const uint32_t k = J.param;
    const uint32_t low = ((1u << k) - 1u) * 0x01010101u, keep = (0xFFu >> k) * 0x01010101u;
    uint32_t w[4];
    load16(J.src, o, J.n, w);  // bytes past the plane read as zero
    uint32_t bad = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      bad |= w[i] & low;
      w[i] = (w[i] >> k) & keep;
    }
    if (bad) atomicOr(&flag[j], 1u);
    store16(J.dst, o, J.n, w);
  }
}

constexpr size_t pxor_lds_bytes(uint32_t w) { return 65536ull * w + 2ull * kPxChunk; }

uint32_t grid_for(uint64_t tiles) { return (uint32_t)std::min<uint64_t>(tiles, kMaxGrid); }

}  // namespace

bool plane_op_supported(uint32_t op, uint32_t param) {
  switch (op) {
    case kPlaneOpNone: return true;
    case kPlaneOpIntDelta: return param == 1 || param == 2 || param == 4 || param == 8;
    case kPlaneOpPredictorXor: return param == 1 || param == 2;
    case kPlaneOpMantissaZeroStrip: return param >= 1 && param <= 7;
    default: return false;
  }
}

int64_t run_plane_ops(DevCtx& ctx, std::vector<PlaneOpJob>& jobs, bool forward, std::vector<uint32_t>* refused) {
  if (refused) refused->assign(jobs.size(), 0);
  if (jobs.empty()) return kOk;
  // the jobs' caller order, for the refusal flags
  std::vector<uint32_t> order(jobs.size());
  for (uint32_t i = 0; i < jobs.size(); ++i) {
    order[i] = i;
    jobs[i].aux = i;  // reset below for IntDelta inverses
  }
  for (const PlaneOpJob& J : jobs)
    if (J.op == kPlaneOpNone || !plane_op_supported(J.op, J.param) || (J.src & 15u) || (J.dst & 15u) ||
        J.n % (J.op == kPlaneOpMantissaZeroStrip ? 1 : J.param))
      return kUnsupported;
  // groups, each one launch (one kernel sequence): IntDelta per width,
  // strip, PredictorXor per width; tiles and sum slots numbered per group
  std::stable_sort(jobs.begin(), jobs.end(), [](const PlaneOpJob& a, const PlaneOpJob& b) {
    return a.op != b.op ? a.op < b.op : a.param < b.param;
  });
  for (uint32_t i = 0; i < jobs.size(); ++i) order[i] = (uint32_t)jobs[i].aux;
  struct Group {
    uint32_t op, param, first, count;
    uint64_t tiles;
  };
  std::vector<Group> groups;
  uint64_t sum_slots = 0;
  for (uint32_t i = 0; i < jobs.size(); ++i) {
    PlaneOpJob& J = jobs[i];
    const uint32_t key_param = J.op == kPlaneOpMantissaZeroStrip ? 0 : J.param;
    if (groups.empty() || groups.back().op != J.op ||
        (groups.back().op != kPlaneOpMantissaZeroStrip && groups.back().param != key_param))
      groups.push_back(Group{J.op, key_param, i, 0, 0});
    Group& G = groups.back();
    const uint64_t nt = (J.n + kTile - 1) / kTile;
    J.tile0 = G.tiles;
    J.aux = J.op == kPlaneOpIntDelta && !forward ? sum_slots : 0;
    if (J.op == kPlaneOpIntDelta && !forward) sum_slots += nt;
    G.tiles += nt;
    ++G.count;
  }
  // jobs, then the PredictorXor job indexes (the jobs themselves, in order)
  const size_t jb = jobs.size() * sizeof(PlaneOpJob);
  const size_t total = jb + jobs.size() * sizeof(uint32_t);
  PTWM_HIP_TRY(ctx.op_jobs.ensure(total));
  PTWM_HIP_TRY(ctx.h_op.ensure(total));
  PTWM_HIP_TRY(ctx.op_sums.ensure(8 * std::max<uint64_t>(sum_slots, jobs.size()) + 8));
  uint32_t* flags = static_cast<uint32_t*>(ctx.op_sums.ptr);  // forward strip refusals
  if (forward) PTWM_HIP_TRY(hipMemsetAsync(flags, 0, 4 * jobs.size(), ctx.stream));
  uint8_t* h = static_cast<uint8_t*>(ctx.h_op.ptr);
  std::memcpy(h, jobs.data(), jb);
  uint32_t* hw = reinterpret_cast<uint32_t*>(h + jb);
  for (uint32_t i = 0; i < jobs.size(); ++i) hw[i] = i;
  hipStream_t s = ctx.stream;
  PTWM_HIP_TRY(hipMemcpyAsync(ctx.op_jobs.ptr, h, total, hipMemcpyHostToDevice, s));
  const PlaneOpJob* dj = static_cast<const PlaneOpJob*>(ctx.op_jobs.ptr);
  const uint32_t* dw = reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(ctx.op_jobs.ptr) + jb);
  uint64_t* sums = static_cast<uint64_t*>(ctx.op_sums.ptr);
  for (const Group& G : groups) {
    const PlaneOpJob* gj = dj + G.first;
    if (G.tiles == 0 && G.op != kPlaneOpPredictorXor) continue;
    if (forward && G.op == kPlaneOpIntDelta) {
#define PTWM_IDELTA_F(W)                                                                                  \
  case W:                                                                                                 \
    hipLaunchKernelGGL(idelta_forward<W>, dim3(grid_for(G.tiles)), dim3(256), 0, s, gj, G.count, G.tiles); \
    break;
      switch (G.param) {
        PTWM_IDELTA_F(1)
        PTWM_IDELTA_F(2)
        PTWM_IDELTA_F(4)
        PTWM_IDELTA_F(8)
        default: return kUnsupported;
      }
#undef PTWM_IDELTA_F
    } else if (forward && G.op == kPlaneOpMantissaZeroStrip) {
      hipLaunchKernelGGL(mzs_forward, dim3(grid_for(G.tiles)), dim3(256), 0, s, gj, G.count, G.tiles,
                         flags + G.first);
    } else if (G.op == kPlaneOpIntDelta) {
#define PTWM_IDELTA(W)                                                                                    \
  case W:                                                                                                 \
    hipLaunchKernelGGL(idelta_sums<W>, dim3(grid_for(G.tiles)), dim3(256), 0, s, gj, G.count, G.tiles, sums); \
    hipLaunchKernelGGL(idelta_scan_sums, dim3(G.count), dim3(256), 0, s, gj, sums);                       \
    hipLaunchKernelGGL(idelta_apply<W>, dim3(grid_for(G.tiles)), dim3(256), 0, s, gj, G.count, G.tiles,  \
                       static_cast<const uint64_t*>(sums));                                               \
    break;
      switch (G.param) {
        PTWM_IDELTA(1)
        PTWM_IDELTA(2)
        PTWM_IDELTA(4)
        PTWM_IDELTA(8)
        default: return kUnsupported;
      }
#undef PTWM_IDELTA
    } else if (G.op == kPlaneOpMantissaZeroStrip) {
      hipLaunchKernelGGL(mzs_inverse, dim3(grid_for(G.tiles)), dim3(256), 0, s, gj, G.count, G.tiles);
    } else if (G.op == kPlaneOpPredictorXor) {
      const void* fn = forward ? (G.param == 1 ? (const void*)pxor_inverse<1, true> : (const void*)pxor_inverse<2, true>)
                               : (G.param == 1 ? (const void*)pxor_inverse<1> : (const void*)pxor_inverse<2>);
      const size_t lds = pxor_lds_bytes(G.param);
      PTWM_HIP_TRY(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
      const uint32_t* which = dw + G.first;
      void* args[] = {&dj, &which};
      PTWM_HIP_TRY(hipLaunchKernel(fn, dim3(G.count), dim3(64), args, lds, s));
    }
    PTWM_HIP_TRY(hipGetLastError());
  }
  if (refused) {
    std::vector<uint32_t> f(jobs.size(), 0);
    PTWM_HIP_TRY(hipMemcpyAsync(f.data(), flags, 4 * jobs.size(), hipMemcpyDeviceToHost, s));
    PTWM_HIP_TRY(hipStreamSynchronize(s));
    for (uint32_t i = 0; i < jobs.size(); ++i) (*refused)[order[i]] = f[i];
  }
  return kOk;
}

}  // namespace ptwm
