// crc_device.h -- CRC-32/ISO-HDLC building blocks shared by the CRC kernels
// (integrity.hip) and the fused decode's CRC of the planes it restores
// (huff_ilv.hip).  Reflected representation: bit 31 - i holds the x^i
// coefficient; a zero-initialised CRC register is linear in the data, and
// advancing it over m zero bytes multiplies it by x^(8m) mod P.
#pragma once

#include "ptwm_common.h"

namespace ptwm {

constexpr uint32_t kCrcPoly = 0xEDB88320u;  // reflected x^32 + x^26 + ... + 1; bit 31 = x^0
constexpr uint32_t kCrcOne = 0x80000000u;   // the polynomial 1
constexpr uint32_t kCrcPiece = 16, kCrcThreads = 256, kCrcTile = kCrcPiece * kCrcThreads;

// Table layout in device memory (words):
//   [0, 1024)     T0..T3: one-byte table and its slicing-by-4 successors
//   [1024, 2048)  S0..S3: byte-sliced advance over kCrcTile zero bytes
//   [2048, 2304)  K[t] = x^(8 * 16 * (255 - t))
//   [2304, 2368)  X[k] = x^(8 * 2^k)
//   [2368, 3392)  byte-sliced advance over 1024 zero bytes (one lane's
//                 stride in a huff_ilv block: 64 lanes x 16 bytes)
//   [3392, 3456)  K64[l] = x^(8 * 16 * (63 - l)): lane l's last piece of a
//                 block to the block's end
constexpr uint32_t kCrcTabS = 1024, kCrcTabK = 2048, kCrcTabX = 2304, kCrcTabS1024 = 2368, kCrcTabK64 = 3392, kCrcTabWords = 3456;

// a * b mod P, reflected representation (bit 31 - i holds the x^i coefficient)
__host__ __device__ inline uint32_t gf2_mulmod(uint32_t a, uint32_t b) {
  uint32_t p = 0;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    p ^= b & (0u - ((a >> (31 - i)) & 1u));
    b = (b >> 1) ^ (kCrcPoly & (0u - (b & 1u)));
  }
  return p;
}

// The same, computed as a short loop: unrolled whole, the compiler keeps
// all 32 shifted multiples of b in registers at once, which in a kernel
// that needs its registers elsewhere costs occupancy.
__device__ __forceinline__ uint32_t gf2_mulmod_seq(uint32_t a, uint32_t b) {
  uint32_t p = 0;
#pragma unroll 4
  for (int i = 0; i < 32; ++i) {
    p ^= b & (0u - ((a >> (31 - i)) & 1u));
    b = (b >> 1) ^ (kCrcPoly & (0u - (b & 1u)));
  }
  return p;
}

// x^(8 n) mod P from the squares table X (X[k] = x^(8 * 2^k))
__host__ __device__ inline uint32_t xpow8(uint64_t n, const uint32_t* X) {
  uint32_t r = kCrcOne;
  for (int k = 0; n; ++k, n >>= 1)
    if (n & 1u) r = gf2_mulmod(r, X[k]);
  return r;
}

__device__ __forceinline__ uint32_t sliced(const uint32_t* L, uint32_t c) {
  return L[c & 255u] ^ L[256 + ((c >> 8) & 255u)] ^ L[512 + ((c >> 16) & 255u)] ^ L[768 + (c >> 24)];
}

// one word through the one-byte tables T0..T3 (T3 takes the first byte)
__device__ __forceinline__ uint32_t crc_word(const uint32_t* T, uint32_t c, uint32_t w) {
  c ^= w;
  return T[768 + (c & 255u)] ^ T[512 + ((c >> 8) & 255u)] ^ T[256 + ((c >> 16) & 255u)] ^ T[c >> 24];
}

__device__ __forceinline__ uint32_t crc_piece(const uint32_t* T, uint32_t c, u32x4 v) {
  c = crc_word(T, c, v.x);
  c = crc_word(T, c, v.y);
  c = crc_word(T, c, v.z);
  return crc_word(T, c, v.w);
}

// ---- the fused decode's CRC, tables at LDS byte address 0 ----
// T0..T3 at words [0, 1024) and the byte-sliced advance over 1024 zero
// bytes at [1024, 2048) (kCrcLdsWords).  With the tables at address 0, an
// entry's address is its index byte times 4, one SDWA shift that picks the
// byte itself, and the table's offset is the load's immediate.
constexpr uint32_t kCrcLdsWords = 2048;

template <int k>
__device__ __forceinline__ uint32_t byte_x4(uint32_t x) {
  uint32_t r;
  if constexpr (k == 0)
    asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0"
        : "=v"(r) : "v"(x));
  else if constexpr (k == 1)
    asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1"
        : "=v"(r) : "v"(x));
  else if constexpr (k == 2)
    asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2"
        : "=v"(r) : "v"(x));
  else
    asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3"
        : "=v"(r) : "v"(x));
  return r;
}

// word kWord of the LDS tables at address 0, plus a byte offset
template <uint32_t kWord>
__device__ __forceinline__ uint32_t lds_tab0(uint32_t byte_off) {
  return *(const __attribute__((address_space(3))) uint32_t*)(uintptr_t)(byte_off + 4u * kWord);
}

// one word through T0..T3 (T3 takes the first byte)
__device__ __forceinline__ uint32_t crc_word_lds0(uint32_t c, uint32_t w) {
  c ^= w;
  return lds_tab0<768>(byte_x4<0>(c)) ^ lds_tab0<512>(byte_x4<1>(c)) ^ lds_tab0<256>(byte_x4<2>(c)) ^
         lds_tab0<0>(byte_x4<3>(c));
}

// acc x^(8 * 1024) xor crc0(piece)
__device__ __forceinline__ uint32_t crc_round_lds0(uint32_t acc, u32x4 v) {
  uint32_t c = crc_word_lds0(0u, v.x);
  c = crc_word_lds0(c, v.y);
  c = crc_word_lds0(c, v.z);
  c = crc_word_lds0(c, v.w);
  return c ^ lds_tab0<1024>(byte_x4<0>(acc)) ^ lds_tab0<1280>(byte_x4<1>(acc)) ^ lds_tab0<1536>(byte_x4<2>(acc)) ^
         lds_tab0<1792>(byte_x4<3>(acc));
}

}  // namespace ptwm
