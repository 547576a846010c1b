// chain_ops.h -- per-word forms of the forward and inverse chains (bit
// reorder + byte/nibble split), shared by the split/merge kernels and the
// plane-CRC kernel.
//
// Bit formulas: split/dtype16.rs:11-25, split/dtype32.rs:13-55,
// split/dtype8.rs:30-62; plane order: transforms/fusion.rs forward
// :35-94,208-255,329-338,431-440.
#pragma once

#include "ptwm_common.h"

namespace ptwm {

__device__ __forceinline__ uint32_t reorder16x2(uint32_t v) {
  return ((v << 1) & 0xFF00FF00u) | ((v >> 8) & 0x00800080u) | (v & 0x007F007Fu);
}
__device__ __forceinline__ uint32_t revert16x2(uint32_t v) {
  return ((v << 8) & 0x80008000u) | ((v >> 1) & 0x7F807F80u) | (v & 0x007F007Fu);
}
__device__ __forceinline__ uint32_t reorder32(uint32_t v) {
  return ((v << 1) & 0xFF000000u) | ((v >> 8) & 0x00800000u) | (v & 0x007FFFFFu);
}
__device__ __forceinline__ uint32_t revert32(uint32_t v) {
  return ((v << 8) & 0x80000000u) | ((v >> 1) & 0x7F800000u) | (v & 0x007FFFFFu);
}
// four fp8 bytes at once
__device__ __forceinline__ uint32_t reorder_e4m3x4(uint32_t v) {
  return ((v & 0x78787878u) << 1) | ((v & 0x80808080u) >> 4) | (v & 0x07070707u);
}
__device__ __forceinline__ uint32_t revert_e4m3x4(uint32_t r) {
  return ((r & 0xF0F0F0F0u) >> 1) | ((r & 0x08080808u) << 4) | (r & 0x07070707u);
}
__device__ __forceinline__ uint32_t reorder_e5m2x4(uint32_t v) {
  return ((v & 0x7C7C7C7Cu) << 1) | ((v & 0x80808080u) >> 5) | (v & 0x03030303u);
}
__device__ __forceinline__ uint32_t revert_e5m2x4(uint32_t r) {
  return ((r & 0xF8F8F8F8u) >> 1) | ((r & 0x04040404u) << 5) | (r & 0x03030303u);
}

// byte interleave: (a0 a1 a2 a3), (b0 b1 b2 b3) -> (a0 b0 a1 b1), (a2 b2 a3 b3)
__device__ __forceinline__ void zip2(uint32_t a, uint32_t b, uint32_t& lo, uint32_t& hi) {
  lo = __builtin_amdgcn_perm(b, a, 0x05010400u);
  hi = __builtin_amdgcn_perm(b, a, 0x07030602u);
}
// inverse of zip2
__device__ __forceinline__ void unzip2(uint32_t lo, uint32_t hi, uint32_t& a, uint32_t& b) {
  a = __builtin_amdgcn_perm(hi, lo, 0x06040200u);  // lo.b0 lo.b2 hi.b0 hi.b2
  b = __builtin_amdgcn_perm(hi, lo, 0x07050301u);
}

// Forward chain of 16 elements: `s` holds the 16 * ratio tensor bytes as
// ratio dwordx4 vectors; plane j's 16 bytes land in out[j].  Chains 1
// (ieee16 split2), 2 (ieee32 split4) and 6 (passthrough).
template <uint32_t kChain>
__device__ __forceinline__ void forward16(const u32x4* s, u32x4* out) {
  if constexpr (kChain == kChainIeee16Split2) {
    uint32_t a[4], b[4];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      unzip2(reorder16x2(s[h].x), reorder16x2(s[h].y), a[2 * h], b[2 * h]);
      unzip2(reorder16x2(s[h].z), reorder16x2(s[h].w), a[2 * h + 1], b[2 * h + 1]);
    }
    out[0] = u32x4_make(a[0], a[1], a[2], a[3]);
    out[1] = u32x4_make(b[0], b[1], b[2], b[3]);
  } else if constexpr (kChain == kChainIeee32Split4) {
    uint32_t o[4][4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t w0 = reorder32(s[k].x), w1 = reorder32(s[k].y), w2 = reorder32(s[k].z), w3 = reorder32(s[k].w);
      const uint32_t t01lo = __builtin_amdgcn_perm(w1, w0, 0x05010400u);
      const uint32_t t01hi = __builtin_amdgcn_perm(w1, w0, 0x07030602u);
      const uint32_t t23lo = __builtin_amdgcn_perm(w3, w2, 0x05010400u);
      const uint32_t t23hi = __builtin_amdgcn_perm(w3, w2, 0x07030602u);
      o[0][k] = __builtin_amdgcn_perm(t23lo, t01lo, 0x05040100u);
      o[1][k] = __builtin_amdgcn_perm(t23lo, t01lo, 0x07060302u);
      o[2][k] = __builtin_amdgcn_perm(t23hi, t01hi, 0x05040100u);
      o[3][k] = __builtin_amdgcn_perm(t23hi, t01hi, 0x07060302u);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) out[j] = u32x4_make(o[j][0], o[j][1], o[j][2], o[j][3]);
  } else {
    out[0] = s[0];
  }
}

// Forward chain of one element: byte of plane j for element i of the tensor
// at device address t.
template <uint32_t kChain>
__device__ __forceinline__ uint8_t forward_byte(uint64_t t, uint64_t i, int j) {
  if constexpr (kChain == kChainIeee16Split2) {
    const uint32_t v = (uint32_t)g_ld<uint8_t>(t + 2 * i) | ((uint32_t)g_ld<uint8_t>(t + 2 * i + 1) << 8);
    return (uint8_t)(reorder16x2(v) >> (8 * j));
  } else if constexpr (kChain == kChainIeee32Split4) {
    uint32_t v = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) v |= (uint32_t)g_ld<uint8_t>(t + 4 * i + b) << (8 * b);
    return (uint8_t)(reorder32(v) >> (8 * j));
  } else {
    return g_ld<uint8_t>(t + i);
  }
}

}  // namespace ptwm
