// ilv_common.h -- device code shared by the GPU-native interleaved plane
// codecs (huff_ilv.hip, rans_ilv.hip): the fused inverse chain (symbol
// transforms and per-group merge), group geometry and memory helpers.
#pragma once

#include "chain_ops.h"
#include "huff_ilv.h"
#include "ptwm_common.h"

namespace ptwm {

// inclusive prefix sum across the 64 lanes of a wavefront
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  const uint32_t lane = threadIdx.x & 63u;
#pragma unroll
  for (uint32_t d = 1; d < 64; d <<= 1) {
    uint32_t t = __shfl_up(v, d, 64);
    if (lane >= d) v += t;
  }
  return v;
}

// Plain global-memory loads (addresses that arrive through LDS would
// otherwise become flat loads).  Payload words are 4-byte aligned (the host
// realigns payloads that are not).
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
__device__ __forceinline__ uint32_t gload_u32(const uint32_t* p) {
  return *(const __attribute__((address_space(1))) uint32_t*)(uintptr_t)p;
}
__device__ __forceinline__ u32x4a4 gload_u32x4(const uint32_t* p) {
  return __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4a4*)(uintptr_t)p);
}
// Streaming (nontemporal) 16-byte load / store and byte access at a device
// address.  Explicitly global: flat accesses would also count against the
// LDS wait counter and stall every table lookup behind them.
__device__ __forceinline__ u32x4 gload_nt16(uint64_t a) {
  return __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4*)(uintptr_t)a);
}
__device__ __forceinline__ void gstore_nt16(uint64_t a, u32x4 v) {
  __builtin_nontemporal_store(v, (__attribute__((address_space(1))) u32x4*)(uintptr_t)a);
}
__device__ __forceinline__ uint32_t gload_u8(uint64_t a) {
  return *(const __attribute__((address_space(1))) uint8_t*)(uintptr_t)a;
}
__device__ __forceinline__ void gstore_u8(uint64_t a, uint32_t v) {
  *(__attribute__((address_space(1))) uint8_t*)(uintptr_t)a = (uint8_t)v;
}

// LDS addresses as plain 32-bit integers: lane bit positions are absolute
// LDS bit addresses, so a window's word address is (q >> 3) & ~3 with no
// base to add, and table bases are constants folded into the ds offsets.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ uint32_t lds_ld32(uint32_t a) {
  return *(const __attribute__((address_space(3))) uint32_t*)(uintptr_t)a;
}
__device__ __forceinline__ uint32_t lds_ld16(uint32_t a) {
  return *(const __attribute__((address_space(3))) uint16_t*)(uintptr_t)a;
}

// Symbol transforms: the per-plane half of each chain's inverse
// (transforms/fusion.rs:150-176, 279-296, 392-399; dtype8.rs:39-62).
enum Xform : uint32_t {
  kXNone = 0,
  kXRot1 = 1,     // IEEE exponent byte e -> (e >> 1) | (e & 1) << 7
  kXHi3 = 2,      // fp8 exponent nibble h -> (h & 0xF) << 3
  kXE4m3Lo = 3,   // E4M3 sign/mantissa nibble l -> (l & 8) << 4 | (l & 7)
  kXE5m2Lo = 4,   // E5M2 sign/mantissa nibble l -> (l & 8) >> 1 | (l & 4) << 5 | (l & 3)
  kXHi4 = 5,      // nibble split high plane h -> (h & 0xF) << 4
  kXLo4 = 6,      // nibble split low plane l -> l & 0xF
};

__device__ __forceinline__ uint32_t xform_byte(uint32_t x, uint32_t s) {
  switch (x) {
    case kXRot1: return ((s >> 1) | (s << 7)) & 0xFFu;
    case kXHi3: return (s & 0xFu) << 3;
    case kXE4m3Lo: return ((s & 8u) << 4) | (s & 7u);
    case kXE5m2Lo: return ((s & 8u) >> 1) | ((s & 4u) << 5) | (s & 3u);
    case kXHi4: return (s & 0xFu) << 4;
    case kXLo4: return s & 0xFu;
    default: return s;
  }
}

// The same transform on 4 packed bytes (raw planes; x is a constant after
// unrolling, so the switch folds away).
__device__ __forceinline__ uint32_t xform_word(uint32_t x, uint32_t v) {
  switch (x) {
    case kXRot1: return ((v >> 1) & 0x7F7F7F7Fu) | ((v << 7) & 0x80808080u);
    case kXHi3: return (v & 0x0F0F0F0Fu) << 3;
    case kXE4m3Lo: return ((v & 0x08080808u) << 4) | (v & 0x07070707u);
    case kXE5m2Lo: return ((v & 0x08080808u) >> 1) | ((v & 0x04040404u) << 5) | (v & 0x03030303u);
    case kXHi4: return (v & 0x0F0F0F0Fu) << 4;
    case kXLo4: return v & 0x0F0F0F0Fu;
    default: return v;
  }
}

// Planes, output bytes per plane byte and the symbol transform of each plane
// (applied by the decode table for coded planes, by xform_word for raw
// ones) per chain.
// Plane bytes back from xform_word's output, for the transforms of the
// chains whose fused decode also computes plane CRCs (kXNone, kXRot1: the
// inverse rotates each byte left by one).
__device__ __forceinline__ uint32_t unxform_word(uint32_t x, uint32_t v) {
  return x == kXRot1 ? ((v << 1) & 0xFEFEFEFEu) | ((v >> 7) & 0x01010101u) : v;
}

template <uint32_t kChain>
struct ChainInfo;
template <> struct ChainInfo<kChainIeee16Split2> {
  static constexpr uint32_t np = 2, ratio = 2;
  static constexpr uint32_t xf[2] = {kXNone, kXRot1};
};
template <> struct ChainInfo<kChainIeee32Split4> {
  static constexpr uint32_t np = 4, ratio = 4;
  static constexpr uint32_t xf[4] = {kXNone, kXNone, kXNone, kXRot1};
};
template <> struct ChainInfo<kChainE4m3Nibble> {
  static constexpr uint32_t np = 2, ratio = 1;
  static constexpr uint32_t xf[2] = {kXHi3, kXE4m3Lo};
};
template <> struct ChainInfo<kChainE5m2Nibble> {
  static constexpr uint32_t np = 2, ratio = 1;
  static constexpr uint32_t xf[2] = {kXHi3, kXE5m2Lo};
};
template <> struct ChainInfo<kChainNibbleSplit> {
  static constexpr uint32_t np = 2, ratio = 1;
  static constexpr uint32_t xf[2] = {kXHi4, kXLo4};
};
template <> struct ChainInfo<kChainPassthrough> {
  static constexpr uint32_t np = 1, ratio = 1;
  static constexpr uint32_t xf[1] = {kXNone};
};

// Merge one group (16 elements; v[p][k] = transformed plane p bytes
// 4k..4k+3) into the output words o[] (ratio * 4 words).  With the exponent
// byte rotated (e' = e >> 1 | (e & 1) << 7), the IEEE inverses of
// fusion.rs:150-176 / 279-296 become a byte interleave plus one bit-select:
// out.lo = mant_lo.7bits | e'.bit7, out.hi = sign | e'.7bits.  The fp8 and
// nibble inverses become a plain OR of the two transformed nibble planes.
template <uint32_t kChain>
__device__ __forceinline__ void merge_group(const uint32_t (&v)[ChainInfo<kChain>::np][4],
                                            uint32_t (&o)[4 * ChainInfo<kChain>::ratio]) {
  if constexpr (kChain == kChainIeee16Split2) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      // a = [m0 e0' m1 e1'], b = [e0' m0 e1' m1] (and the same for bytes 2, 3)
      const uint32_t a0 = __builtin_amdgcn_perm(v[1][k], v[0][k], 0x05010400u);
      const uint32_t b0 = __builtin_amdgcn_perm(v[1][k], v[0][k], 0x01050004u);
      const uint32_t a1 = __builtin_amdgcn_perm(v[1][k], v[0][k], 0x07030602u);
      const uint32_t b1 = __builtin_amdgcn_perm(v[1][k], v[0][k], 0x03070206u);
      o[2 * k] = (a0 & 0x7F7F7F7Fu) | (b0 & 0x80808080u);
      o[2 * k + 1] = (a1 & 0x7F7F7F7Fu) | (b1 & 0x80808080u);
    }
  } else if constexpr (kChain == kChainIeee32Split4) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t ab_lo, ab_hi, cd_lo, cd_hi;
      zip2(v[0][k], v[1][k], ab_lo, ab_hi);
      zip2(v[2][k], v[3][k], cd_lo, cd_hi);
      // a = [b0 b1 b2 e'], b = [b0 b1 e' b2]: keep a's 0x7F7FFFFF bits
      const uint32_t a[4] = {__builtin_amdgcn_perm(cd_lo, ab_lo, 0x05040100u),
                             __builtin_amdgcn_perm(cd_lo, ab_lo, 0x07060302u),
                             __builtin_amdgcn_perm(cd_hi, ab_hi, 0x05040100u),
                             __builtin_amdgcn_perm(cd_hi, ab_hi, 0x07060302u)};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t b = __builtin_amdgcn_perm(a[i], a[i], 0x02030100u);
        o[4 * k + i] = (a[i] & 0x7F7FFFFFu) | (b & 0x80800000u);
      }
    }
  } else if constexpr (kChain == kChainPassthrough) {
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = v[0][k];
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = v[0][k] | v[1][k];
  }
}

// Symbols of plane positions [pos, pos + 16) clipped to n.
template <bool kTail>
__device__ __forceinline__ uint32_t group_count(uint64_t pos, uint64_t n) {
  if (!kTail) return kIlvGroup;
  return pos < n ? (uint32_t)(n - pos < kIlvGroup ? n - pos : kIlvGroup) : 0u;
}

// Packed-nibble payloads (tag 2 of both GPU-native codecs):
// [2][n u32][0 0 0][ceil(n / 2) bytes], byte i = s[2i] | s[2i+1] << 4, the
// high nibble of the last byte 0 when n is odd.
// pay: the payload's first 8 bytes; last: its last byte.
__device__ __forceinline__ bool packed_header_ok(const uint8_t* pay, uint64_t len, uint64_t n, uint32_t last) {
  if (len < kPackedHeadBytes || pay[5] || pay[6] || pay[7]) return false;
  const uint64_t pn = (uint64_t)pay[1] | ((uint64_t)pay[2] << 8) | ((uint64_t)pay[3] << 16) | ((uint64_t)pay[4] << 24);
  if (pn != n || len != kPackedHeadBytes + (n + 1) / 2) return false;
  return !(n & 1u) || (last >> 4) == 0;
}

// The 16 symbols of the group at plane position pos (count of them inside
// the plane) of a stored plane at `base`: bytes, or packed nibbles (base =
// payload + 8, 4-byte aligned) expanded to one symbol per byte.
__device__ __forceinline__ void load_group(uint64_t base, bool packed, uint64_t pos, uint32_t count,
                                           uint32_t (&x)[4]) {
  if (!packed) {
    const uint64_t a = base + pos;
    if (count == kIlvGroup && (base & 15u) == 0) {
      const u32x4 w = gload_nt16(a);
      x[0] = w.x;
      x[1] = w.y;
      x[2] = w.z;
      x[3] = w.w;
    } else {
      x[0] = x[1] = x[2] = x[3] = 0;
      for (uint32_t k = 0; k < count; ++k) x[k >> 2] |= gload_u8(a + k) << (8 * (k & 3));
    }
    return;
  }
  const uint64_t a = base + pos / 2;  // pos is a multiple of 16
  uint32_t w[2] = {0, 0};
  if (count == kIlvGroup && (base & 3u) == 0) {
    w[0] = g_ld<uint32_t>(a);
    w[1] = g_ld<uint32_t>(a + 4);
  } else {
    for (uint32_t k = 0; k < (count + 1) / 2; ++k) w[k >> 2] |= gload_u8(a + k) << (8 * (k & 3));
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    // even nibbles and odd nibbles, then interleaved back into symbol order
    zip2(w[h] & 0x0F0F0F0Fu, (w[h] >> 4) & 0x0F0F0F0Fu, x[2 * h], x[2 * h + 1]);
  }
}

// Fast path of the raw-plane loads (full groups of planes under 4 GiB, bases
// aligned as raw_aligned requires): one buffer load per plane per round,
// issued for every plane unconditionally (a coded plane has an empty
// resource: loads past num_records return zeros without a memory access),
// so each round issues a fixed sequence of memory operations and the wait
// before the consumer (expand_group) leaves the stores issued after the
// load in flight.  A packed plane's 16-byte load at pos / 2 uses its first
// 8 bytes; the rest may lie past the plane and then reads as zeros.
__device__ __forceinline__ bool raw_aligned(uint64_t base, bool packed) {
  return (base & (packed ? 7u : 15u)) == 0;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t plane_rsrc(uint64_t base, uint32_t bytes) {
  // raw buffer: stride 0, 32-bit data format word of the gfx9 family
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// live == false: a load at offset `bytes`, past the resource (zeros, no
// memory access), keeping the sequence of memory operations fixed.
__device__ __forceinline__ void load_group_fast(uint64_t base, uint32_t bytes, bool packed, uint32_t pos, bool live,
                                                uint32_t (&x)[4]) {
  const uint32_t off = live ? (packed ? pos / 2 : pos) : bytes;
  const u32x4 w = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(plane_rsrc(base, bytes), off, 0, 0));
  x[0] = w.x;
  x[1] = w.y;
  x[2] = w.z;
  x[3] = w.w;
}

// A vector memory operation that does nothing: a buffer store to an empty
// resource (num_records 0), discarded without a memory access.  The fast
// decode loop issues one per output store after its first raw loads, so
// that the loop is entered with the same count of memory operations behind
// its loads as every later round has (the raw loads, then the stores); the
// compiler's wait before the consumer then leaves the stores in flight.
// (k: distinct offsets, so that repeated calls are not merged)
__device__ __forceinline__ void vmem_nop(uint64_t base, uint32_t k) {
  __builtin_amdgcn_raw_buffer_store_b32(0u, plane_rsrc(base, 0), 4 * k, 0, (int)0x80000000u);  // volatile: kept apart
}

// Store of the RATIO * 16 output bytes of each lane's group in a full round
// (all 64 lanes storing whole, adjacent groups).  Plain (temporal) stores,
// so that the L2 combines the pieces of a line; with RATIO 2 the lanes of
// each quad first exchange halves (DPP quad permutes), so that every store
// instruction writes whole 64-byte segments: lane q of the quad at qb
// stores bytes [16 q, 16 q + 16) of [qb, qb + 64) and then of
// [qb + 64, qb + 128), taken from lane q / 2, resp. 2 + q / 2, half q & 1.
template <uint32_t RATIO>
__device__ __forceinline__ void store_group_full(uint64_t dst, uint32_t lane, const uint32_t (&o)[4 * RATIO]) {
  if constexpr (RATIO == 2) {
    const uint32_t q = lane & 3u;
    const uint64_t qb = dst - 32u * q;
    uint32_t a0[4], a1[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      // quad_perm [0,0,1,1] = 0x50, [2,2,3,3] = 0xFA
      const uint32_t x0 = __builtin_amdgcn_mov_dpp(o[d], 0x50, 0xF, 0xF, false);
      const uint32_t y0 = __builtin_amdgcn_mov_dpp(o[4 + d], 0x50, 0xF, 0xF, false);
      const uint32_t x1 = __builtin_amdgcn_mov_dpp(o[d], 0xFA, 0xF, 0xF, false);
      const uint32_t y1 = __builtin_amdgcn_mov_dpp(o[4 + d], 0xFA, 0xF, 0xF, false);
      a0[d] = (q & 1u) ? y0 : x0;
      a1[d] = (q & 1u) ? y1 : x1;
    }
    g_st<u32x4>(qb + 16u * q, u32x4_make(a0[0], a0[1], a0[2], a0[3]));
    g_st<u32x4>(qb + 64u + 16u * q, u32x4_make(a1[0], a1[1], a1[2], a1[3]));
  } else {
#pragma unroll
    for (uint32_t k = 0; k < RATIO; ++k)
      g_st<u32x4>(dst + 16 * k, u32x4_make(o[4 * k], o[4 * k + 1], o[4 * k + 2], o[4 * k + 3]));
  }
}

// Error bits into a tensor's status word.  The status words live in
// host-coherent (pinned) memory that the host reads after the stream has
// drained: system scope, a vector atomic.
__device__ __forceinline__ void status_or(uint32_t* w, uint32_t v) {
  __hip_atomic_fetch_or(w, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// OR of a status word (bits 0..7) over the wavefront's active lanes, so
// that one lane reports it: per-lane atomics on one status word serialise.
__device__ __forceinline__ uint32_t wave_or_status(uint32_t v) {
  uint32_t r = 0;
#pragma unroll
  for (uint32_t b = 0; b < 8; ++b)
    if (__ballot((v >> b) & 1u)) r |= 1u << b;
  return r;
}

// The 16 symbols of a group loaded by load_group_fast, one per byte.  Reads
// all four words whatever `packed` is (selects, no branch), so that every
// path waits for the load at this point and nowhere later.
__device__ __forceinline__ void expand_group(bool packed, const uint32_t (&x)[4], uint32_t (&v)[4]) {
  uint32_t u[4];
  zip2(x[0] & 0x0F0F0F0Fu, (x[0] >> 4) & 0x0F0F0F0Fu, u[0], u[1]);
  zip2(x[1] & 0x0F0F0F0Fu, (x[1] >> 4) & 0x0F0F0F0Fu, u[2], u[3]);
#pragma unroll
  for (int k = 0; k < 4; ++k) v[k] = packed ? u[k] : x[k];
}

}  // namespace ptwm
