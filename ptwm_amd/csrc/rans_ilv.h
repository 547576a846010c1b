// rans_ilv.h -- descriptors and launchers of the GPU-native interleaved rANS
// plane codec (format and design notes in rans_ilv.hip).
#pragma once

#include "huff_ilv.h"
#include "ptwm_common.h"

namespace ptwm {

constexpr uint32_t kRilvTableBytes = 8192;   // 2048 u32 entries per coded plane
constexpr uint32_t kRilvProbBits = 11;
constexpr uint32_t kRilvL = 1u << 16;         // state lower bound; words are 16 bits
constexpr uint32_t kRilvBlockHead = 260;      // [nw u32][64 x u32 states]
constexpr uint32_t kRilvMaxLds = 81920;
// Payload bytes read per native plane at a tensor's start (tag, n, max_sym,
// 256 frequencies, padding), kept in the staging area.
constexpr uint32_t kRilvHeadWords = 132;

// status bits (per tensor), in addition to kIlvErrHeader / kIlvErrBlock
constexpr uint32_t kRilvErrState = 8;  // words left over / missing or a final state != 2^16

// Encoder: per coded plane, 256 symbol entries f | cum << 16 (normalised
// frequencies, rans/compress.rs:72-122).
struct RilvEncBlock {
  uint64_t dst;     // device address of the block (nw first)
  uint32_t plane;   // index into the IlvEncPlane array
  uint32_t block;   // block index within the plane
};

// Fused decode of the tensors tix[0..m) (indexes into `tensors`, all of
// chain `chain`, coded planes rans_ilv).  Same tiling and persistence as
// launch_ilv_decode; stage_words: LDS words per wavefront for the block's
// words (multiple of 4), blocks needing more read their words from global
// memory.
hipError_t launch_rilv_decode(uint32_t chain, const IlvTensor* tensors, const uint32_t* tix, const uint32_t* tpre,
                              uint32_t m, uint32_t grid, uint32_t* status, uint32_t n_slots, uint32_t stage_words,
                              hipStream_t stream);
size_t rilv_decode_lds_bytes(uint32_t chain, uint32_t n_slots, uint32_t stage_words);
hipError_t rilv_decode_occupancy(uint32_t chain, uint32_t n_slots, uint32_t stage_words, int* wg_per_cu);

// Encoder passes over blocks: word counts (block_words[i]), then the blocks.
hipError_t launch_rilv_size(const IlvEncPlane* planes, const RilvEncBlock* blocks, uint32_t n_blocks,
                            const uint32_t* syms, uint32_t* block_words, hipStream_t stream);
hipError_t launch_rilv_encode(const IlvEncPlane* planes, const RilvEncBlock* blocks, uint32_t n_blocks,
                              const uint32_t* syms, const uint32_t* block_words, hipStream_t stream);

}  // namespace ptwm
