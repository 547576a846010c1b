// transform.hip -- fused bit-reorder + byte/nibble split and merge on gfx950.
//
// Streaming HBM->HBM passes: every lane moves 16 elements per step with
// dwordx4 loads/stores, so each wavefront instruction covers a contiguous
// 1 KiB (planes) to 4 KiB (fp32 tensor) span.  Grid-stride, launched with
// enough workgroups to cover all 256 CUs several times.
//
// Semantics follow transforms/fusion.rs (forward :35-94,208-255,329-338,
// 431-440; inverse :127-194,261-315,376-399,478-501), NibbleSplit
// (transforms/nibble_split.rs:72-120) and BytePassthrough.
#include "chain_ops.h"
#include "ptwm_common.h"

namespace ptwm {

namespace {

struct Planes {
  uint8_t* p[4];
};

}  // namespace

// ---------------------------------------------------------------------------
// inverse (merge): planes -> tensor
// ---------------------------------------------------------------------------

// bf16/fp16: 16 elements per lane step: 16 B from each plane -> 32 B out.
__global__ void __launch_bounds__(256) merge_ieee16_kernel(const uint8_t* __restrict__ p0,
                                                           const uint8_t* __restrict__ p1,
                                                           uint8_t* __restrict__ out, uint64_t n) {
  const uint64_t nvec = n / 16;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t v = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; v < nvec; v += stride) {
    u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p0) + v);
    u32x4 b = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p1) + v);
    u32x4 o0, o1;
    uint32_t lo, hi;
    zip2(a.x, b.x, lo, hi); o0.x = revert16x2(lo); o0.y = revert16x2(hi);
    zip2(a.y, b.y, lo, hi); o0.z = revert16x2(lo); o0.w = revert16x2(hi);
    zip2(a.z, b.z, lo, hi); o1.x = revert16x2(lo); o1.y = revert16x2(hi);
    zip2(a.w, b.w, lo, hi); o1.z = revert16x2(lo); o1.w = revert16x2(hi);
    u32x4* o = reinterpret_cast<u32x4*>(out) + 2 * v;
    __builtin_nontemporal_store(o0, o);
    __builtin_nontemporal_store(o1, o + 1);
  }
  // tail elements (< 16), including an odd trailing element (fusion.rs:165-176)
  if (blockIdx.x == 0) {
    for (uint64_t i = nvec * 16 + threadIdx.x; i < n; i += blockDim.x) {
      uint32_t r = (uint32_t)p0[i] | ((uint32_t)p1[i] << 8);
      uint32_t v = revert16x2(r);
      out[2 * i] = (uint8_t)v;
      out[2 * i + 1] = (uint8_t)(v >> 8);
    }
  }
}

// fp32: 4 planes x 16 B -> 64 B out.
__global__ void __launch_bounds__(256) merge_ieee32_kernel(const uint8_t* __restrict__ p0,
                                                           const uint8_t* __restrict__ p1,
                                                           const uint8_t* __restrict__ p2,
                                                           const uint8_t* __restrict__ p3,
                                                           uint8_t* __restrict__ out, uint64_t n) {
  const uint64_t nvec = n / 16;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t v = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; v < nvec; v += stride) {
    u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p0) + v);
    u32x4 b = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p1) + v);
    u32x4 c = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p2) + v);
    u32x4 d = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p3) + v);
    const uint32_t av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
    const uint32_t cv[4] = {c.x, c.y, c.z, c.w}, dv[4] = {d.x, d.y, d.z, d.w};
    u32x4* o = reinterpret_cast<u32x4*>(out) + 4 * v;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t ab_lo, ab_hi, cd_lo, cd_hi;
      zip2(av[k], bv[k], ab_lo, ab_hi);  // a0 b0 a1 b1 | a2 b2 a3 b3
      zip2(cv[k], dv[k], cd_lo, cd_hi);
      u32x4 w;
      w.x = revert32(__builtin_amdgcn_perm(cd_lo, ab_lo, 0x05040100u));  // a0 b0 c0 d0
      w.y = revert32(__builtin_amdgcn_perm(cd_lo, ab_lo, 0x07060302u));  // a1 b1 c1 d1
      w.z = revert32(__builtin_amdgcn_perm(cd_hi, ab_hi, 0x05040100u));
      w.w = revert32(__builtin_amdgcn_perm(cd_hi, ab_hi, 0x07060302u));
      __builtin_nontemporal_store(w, o + k);
    }
  }
  if (blockIdx.x == 0) {
    for (uint64_t i = nvec * 16 + threadIdx.x; i < n; i += blockDim.x) {
      uint32_t r = (uint32_t)p0[i] | ((uint32_t)p1[i] << 8) | ((uint32_t)p2[i] << 16) | ((uint32_t)p3[i] << 24);
      uint32_t v = revert32(r);
      out[4 * i] = (uint8_t)v;
      out[4 * i + 1] = (uint8_t)(v >> 8);
      out[4 * i + 2] = (uint8_t)(v >> 16);
      out[4 * i + 3] = (uint8_t)(v >> 24);
    }
  }
}

// nibble planes: hi/lo 16 B each -> 16 B out; mode 0 plain NibbleSplit,
// 1 E4M3 revert, 2 E5M2 revert.  High bits of plane bytes are masked
// (nibble_split.rs:115-120).
template <int kMode>
__global__ void __launch_bounds__(256) merge_nibble_kernel(const uint8_t* __restrict__ hi,
                                                            const uint8_t* __restrict__ lo,
                                                            uint8_t* __restrict__ out, uint64_t n) {
  const uint64_t nvec = n / 16;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  auto f = [](uint32_t h, uint32_t l) -> uint32_t {
    uint32_t r = ((h & 0x0F0F0F0Fu) << 4) | (l & 0x0F0F0F0Fu);
    if (kMode == 1) return revert_e4m3x4(r);
    if (kMode == 2) return revert_e5m2x4(r);
    return r;
  };
  for (uint64_t v = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; v < nvec; v += stride) {
    u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(hi) + v);
    u32x4 b = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(lo) + v);
    u32x4 o;
    o.x = f(a.x, b.x); o.y = f(a.y, b.y); o.z = f(a.z, b.z); o.w = f(a.w, b.w);
    __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(out) + v);
  }
  if (blockIdx.x == 0) {
    for (uint64_t i = nvec * 16 + threadIdx.x; i < n; i += blockDim.x) out[i] = (uint8_t)f(hi[i], lo[i]);
  }
}

// ---------------------------------------------------------------------------
// forward (split): tensor -> planes
// ---------------------------------------------------------------------------

__global__ void __launch_bounds__(256) split_ieee16_kernel(const uint8_t* __restrict__ in,
                                                           uint8_t* __restrict__ p0,
                                                           uint8_t* __restrict__ p1, uint64_t n) {
  const uint64_t nvec = n / 16;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t v = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; v < nvec; v += stride) {
    const u32x4* s = reinterpret_cast<const u32x4*>(in) + 2 * v;
    u32x4 x0 = __builtin_nontemporal_load(s), x1 = __builtin_nontemporal_load(s + 1);
    uint32_t a0, b0, a1, b1, a2, b2, a3, b3;
    unzip2(reorder16x2(x0.x), reorder16x2(x0.y), a0, b0);
    unzip2(reorder16x2(x0.z), reorder16x2(x0.w), a1, b1);
    unzip2(reorder16x2(x1.x), reorder16x2(x1.y), a2, b2);
    unzip2(reorder16x2(x1.z), reorder16x2(x1.w), a3, b3);
    u32x4 a = u32x4_make(a0, a1, a2, a3), b = u32x4_make(b0, b1, b2, b3);
    __builtin_nontemporal_store(a, reinterpret_cast<u32x4*>(p0) + v);
    __builtin_nontemporal_store(b, reinterpret_cast<u32x4*>(p1) + v);
  }
  if (blockIdx.x == 0) {
    for (uint64_t i = nvec * 16 + threadIdx.x; i < n; i += blockDim.x) {
      uint32_t v = (uint32_t)in[2 * i] | ((uint32_t)in[2 * i + 1] << 8);
      uint32_t r = reorder16x2(v);
      p0[i] = (uint8_t)r;
      p1[i] = (uint8_t)(r >> 8);
    }
  }
}

__global__ void __launch_bounds__(256) split_ieee32_kernel(const uint8_t* __restrict__ in,
                                                           uint8_t* __restrict__ p0, uint8_t* __restrict__ p1,
                                                           uint8_t* __restrict__ p2, uint8_t* __restrict__ p3,
                                                           uint64_t n) {
  const uint64_t nvec = n / 16;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t v = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; v < nvec; v += stride) {
    const u32x4* s = reinterpret_cast<const u32x4*>(in) + 4 * v;
    uint32_t o[4][4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      u32x4 x = __builtin_nontemporal_load(s + k);
      uint32_t w0 = reorder32(x.x), w1 = reorder32(x.y), w2 = reorder32(x.z), w3 = reorder32(x.w);
      // transpose 4x4 bytes: plane j gets byte j of w0..w3
      uint32_t t01lo = __builtin_amdgcn_perm(w1, w0, 0x05010400u);  // w0b0 w1b0 w0b1 w1b1
      uint32_t t01hi = __builtin_amdgcn_perm(w1, w0, 0x07030602u);  // w0b2 w1b2 w0b3 w1b3
      uint32_t t23lo = __builtin_amdgcn_perm(w3, w2, 0x05010400u);
      uint32_t t23hi = __builtin_amdgcn_perm(w3, w2, 0x07030602u);
      o[0][k] = __builtin_amdgcn_perm(t23lo, t01lo, 0x05040100u);
      o[1][k] = __builtin_amdgcn_perm(t23lo, t01lo, 0x07060302u);
      o[2][k] = __builtin_amdgcn_perm(t23hi, t01hi, 0x05040100u);
      o[3][k] = __builtin_amdgcn_perm(t23hi, t01hi, 0x07060302u);
    }
    uint8_t* dstp[4] = {p0, p1, p2, p3};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_nontemporal_store(u32x4_make(o[j][0], o[j][1], o[j][2], o[j][3]),
                                  reinterpret_cast<u32x4*>(dstp[j]) + v);
  }
  if (blockIdx.x == 0) {
    for (uint64_t i = nvec * 16 + threadIdx.x; i < n; i += blockDim.x) {
      uint32_t v = (uint32_t)in[4 * i] | ((uint32_t)in[4 * i + 1] << 8) | ((uint32_t)in[4 * i + 2] << 16) |
                   ((uint32_t)in[4 * i + 3] << 24);
      uint32_t r = reorder32(v);
      p0[i] = (uint8_t)r; p1[i] = (uint8_t)(r >> 8); p2[i] = (uint8_t)(r >> 16); p3[i] = (uint8_t)(r >> 24);
    }
  }
}

template <int kMode>
__global__ void __launch_bounds__(256) split_nibble_kernel(const uint8_t* __restrict__ in,
                                                            uint8_t* __restrict__ hi,
                                                            uint8_t* __restrict__ lo, uint64_t n) {
  const uint64_t nvec = n / 16;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  auto f = [](uint32_t v) -> uint32_t {
    if (kMode == 1) return reorder_e4m3x4(v);
    if (kMode == 2) return reorder_e5m2x4(v);
    return v;
  };
  for (uint64_t v = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; v < nvec; v += stride) {
    u32x4 x = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(in) + v);
    uint32_t r0 = f(x.x), r1 = f(x.y), r2 = f(x.z), r3 = f(x.w);
    u32x4 h = u32x4_make((r0 >> 4) & 0x0F0F0F0Fu, (r1 >> 4) & 0x0F0F0F0Fu, (r2 >> 4) & 0x0F0F0F0Fu,
                         (r3 >> 4) & 0x0F0F0F0Fu);
    u32x4 l = u32x4_make(r0 & 0x0F0F0F0Fu, r1 & 0x0F0F0F0Fu, r2 & 0x0F0F0F0Fu, r3 & 0x0F0F0F0Fu);
    __builtin_nontemporal_store(h, reinterpret_cast<u32x4*>(hi) + v);
    __builtin_nontemporal_store(l, reinterpret_cast<u32x4*>(lo) + v);
  }
  if (blockIdx.x == 0) {
    for (uint64_t i = nvec * 16 + threadIdx.x; i < n; i += blockDim.x) {
      uint32_t r = f(in[i]);
      hi[i] = (uint8_t)((r >> 4) & 0x0F);
      lo[i] = (uint8_t)(r & 0x0F);
    }
  }
}

__global__ void __launch_bounds__(256) copy_kernel(const uint8_t* __restrict__ in, uint8_t* __restrict__ out,
                                                   uint64_t n) {
  const uint64_t nvec = n / 16;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t v = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; v < nvec; v += stride)
    __builtin_nontemporal_store(__builtin_nontemporal_load(reinterpret_cast<const u32x4*>(in) + v),
                                reinterpret_cast<u32x4*>(out) + v);
  if (blockIdx.x == 0)
    for (uint64_t i = nvec * 16 + threadIdx.x; i < n; i += blockDim.x) out[i] = in[i];
}

static inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

static inline dim3 stream_grid(uint64_t nvec) {
  // 256 CUs x 8 workgroups keeps every CU busy; fewer for small inputs.
  uint64_t blocks = (nvec + 255) / 256;
  if (blocks > 2048) blocks = 2048;
  if (blocks < 1) blocks = 1;
  return dim3((uint32_t)blocks);
}

// planes: n_planes pointers of plane_len bytes each; out: tensor bytes.
// Returns hipErrorInvalidValue for pointers that break the 16-byte alignment
// the vector path assumes (all allocations this library makes are aligned).
hipError_t launch_merge(uint32_t chain, const uint8_t* const* planes, uint64_t plane_len, uint8_t* out,
                        hipStream_t stream) {
  const uint64_t nvec = plane_len / 16;
  dim3 grid = stream_grid(nvec), block(256);
  bool al = aligned16(out);
  int np = chain == kChainIeee32Split4 ? 4 : (chain == kChainPassthrough ? 1 : 2);
  for (int i = 0; i < np; ++i) al = al && aligned16(planes[i]);
  if (!al) return hipErrorInvalidValue;
  switch (chain) {
    case kChainIeee16Split2:
      hipLaunchKernelGGL(merge_ieee16_kernel, grid, block, 0, stream, planes[0], planes[1], out, plane_len);
      break;
    case kChainIeee32Split4:
      hipLaunchKernelGGL(merge_ieee32_kernel, grid, block, 0, stream, planes[0], planes[1], planes[2], planes[3],
                         out, plane_len);
      break;
    case kChainE4m3Nibble:
      hipLaunchKernelGGL(merge_nibble_kernel<1>, grid, block, 0, stream, planes[0], planes[1], out, plane_len);
      break;
    case kChainE5m2Nibble:
      hipLaunchKernelGGL(merge_nibble_kernel<2>, grid, block, 0, stream, planes[0], planes[1], out, plane_len);
      break;
    case kChainNibbleSplit:
      hipLaunchKernelGGL(merge_nibble_kernel<0>, grid, block, 0, stream, planes[0], planes[1], out, plane_len);
      break;
    case kChainPassthrough:
      hipLaunchKernelGGL(copy_kernel, grid, block, 0, stream, planes[0], out, plane_len);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_split(uint32_t chain, const uint8_t* in, uint64_t plane_len, uint8_t* const* planes,
                        hipStream_t stream) {
  const uint64_t nvec = plane_len / 16;
  dim3 grid = stream_grid(nvec), block(256);
  bool al = aligned16(in);
  int np = chain == kChainIeee32Split4 ? 4 : (chain == kChainPassthrough ? 1 : 2);
  for (int i = 0; i < np; ++i) al = al && aligned16(planes[i]);
  if (!al) return hipErrorInvalidValue;
  switch (chain) {
    case kChainIeee16Split2:
      hipLaunchKernelGGL(split_ieee16_kernel, grid, block, 0, stream, in, planes[0], planes[1], plane_len);
      break;
    case kChainIeee32Split4:
      hipLaunchKernelGGL(split_ieee32_kernel, grid, block, 0, stream, in, planes[0], planes[1], planes[2],
                         planes[3], plane_len);
      break;
    case kChainE4m3Nibble:
      hipLaunchKernelGGL(split_nibble_kernel<1>, grid, block, 0, stream, in, planes[0], planes[1], plane_len);
      break;
    case kChainE5m2Nibble:
      hipLaunchKernelGGL(split_nibble_kernel<2>, grid, block, 0, stream, in, planes[0], planes[1], plane_len);
      break;
    case kChainNibbleSplit:
      hipLaunchKernelGGL(split_nibble_kernel<0>, grid, block, 0, stream, in, planes[0], planes[1], plane_len);
      break;
    case kChainPassthrough:
      hipLaunchKernelGGL(copy_kernel, grid, block, 0, stream, in, planes[0], plane_len);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_copy(const uint8_t* in, uint8_t* out, uint64_t n, hipStream_t stream) {
  if (!aligned16(in) || !aligned16(out)) return hipMemcpyAsync(out, in, n, hipMemcpyDeviceToDevice, stream);
  hipLaunchKernelGGL(copy_kernel, stream_grid(n / 16), dim3(256), 0, stream, in, out, n);
  return hipGetLastError();
}

}  // namespace ptwm
