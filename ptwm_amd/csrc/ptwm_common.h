// ptwm_common.h -- shared definitions for the MI355X plane-codec library.
//
// Error codes follow the reference native ABI return convention
// (crates/ptwm-core/src/flavor/native.rs:634-657): >= 0 bytes written,
// -1 InvalidInput, -2 BufferTooSmall, -3 MissingCapability,
// -4 MissingNativeDep, -5 Unsupported, anything else InternalError.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "codes.h"

namespace ptwm {

// Native 128-bit vector (dwordx4 loads/stores; usable with the nontemporal
// builtins, unlike HIP's uint4 struct).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__host__ __device__ inline u32x4 u32x4_make(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  u32x4 r = {a, b, c, d};
  return r;
}

// Global-memory accesses in address space 1.  Generic (flat) accesses also
// count against the LDS wait counter, so a kernel that mixes LDS lookups
// with flat loads or stores waits for memory on every LDS use.
template <typename T>
__device__ __forceinline__ T g_ld(uint64_t a) {
  return *(const __attribute__((address_space(1))) T*)(uintptr_t)a;
}
template <typename T>
__device__ __forceinline__ void g_st(uint64_t a, T v) {
  *(__attribute__((address_space(1))) T*)(uintptr_t)a = v;
}
__device__ __forceinline__ u32x4 g_ld_nt16(uint64_t a) {
  return __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4*)(uintptr_t)a);
}

// Per-job decode status written by the device (0 = ok).
enum DecodeStatus : uint32_t {
  kStOk = 0,
  kStBadFrame = 1,       // chunk frame truncated / state_len past the end
  kStBadTag = 2,         // tag byte not 0/1 or payload empty
  kStBadLength = 3,      // declared length disagrees with the chunk table / cap
  kStBadHeader = 4,      // weights / frequency table / jump table invalid
  kStBadStream = 5,      // bitstream inconsistent (reference decoder errors)
  kStDeferred = 6,       // header parsed, streams handed to the parallel Huffman path
  kStFallback = 7,       // parallel path declined the payload: decode it on the exact path
  kStUnsettled = 8,      // parallel path: wavefront boundaries not settled by the queued fix passes
  kStNotRun = 0xFFFFFFFFu,
};

// One independently coded unit: a whole plane payload, or one chunk frame
// of a chunked plane (compressor.rs:316-321 frame: [ver u8][state_len u32]
// [state][payload]).  64 bytes so the array is naturally aligned.
struct DecodeJob {
  uint64_t src;       // device address of the payload (or of the chunk frame)
  uint64_t src_len;   // bytes available at src
  uint64_t dst;       // device address of the decoded bytes
  uint64_t dst_len;   // exact decoded size expected (chunk table decoded_size)
  uint32_t codec;     // kCodec*
  uint32_t framed;    // 1: src starts with a chunk frame header
  uint32_t sync_id;   // 0, or 1 + slot of a Huffman payload whose streams go to the parallel path
  uint32_t sync_sub0; // first subsequence slot of that payload
  uint32_t pad[4];     // Order1ScaleAC: its state (o1sac_device.hip); parallel-path Huffman: pad[3] = subsequence bits
};
static_assert(sizeof(DecodeJob) == 64, "DecodeJob layout");

#define PTWM_HIP_TRY(expr)                      \
  do {                                          \
    hipError_t _e = (expr);                     \
    if (_e != hipSuccess) return ::ptwm::kInternal; \
  } while (0)

}  // namespace ptwm
