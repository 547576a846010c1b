// huff_ilv.h -- descriptors and launchers of the GPU-native interleaved
// Huffman codec (format and design notes in huff_ilv.hip).
#pragma once

#include "ptwm_common.h"

namespace ptwm {

constexpr uint32_t kIlvBlock = 16384;   // symbols per block (one wavefront)
constexpr uint32_t kIlvLanes = 64;
constexpr uint32_t kIlvGroup = 16;      // symbols per lane per round
constexpr uint32_t kIlvRounds = kIlvBlock / (kIlvLanes * kIlvGroup);  // 16
constexpr uint32_t kIlvBlocksPerTile = 4;   // blocks per tile (one per wavefront)
constexpr uint32_t kIlvStageSpare = 96;     // spare LDS words after the staging area
constexpr uint32_t kIlvMaxLds = 81920;      // LDS budget of one decode workgroup (2 per CU)
constexpr uint32_t kMaxGridY = 65535;       // launches with one plane or job per gridDim.y slot are sliced

// status bits (per tensor)
constexpr uint32_t kIlvErrHeader = 1;   // tag / length / weights / table bounds
constexpr uint32_t kIlvErrBlock = 2;    // block offsets or lane word counts inconsistent
constexpr uint32_t kIlvErrLane = 4;     // a lane's word count disagrees with its codes
// Not an input error: a coded plane found no LDS table slot in this launch
// (the host reserves slots for the planes whose payload length is neither
// the stored nor the packed length) and the tensor is decoded again with a
// slot for every plane.
constexpr uint32_t kIlvRetrySlots = 16;

// Payload bytes read per native plane at a tensor's start (tag, n, weights
// header: at most 135), kept in the staging area.
constexpr uint32_t kIlvHeadWords = 36;

struct IlvPlane {
  uint64_t base;   // coded: payload address; raw: plane bytes (16-byte aligned)
  uint64_t len;    // coded: payload length
  uint32_t coded;  // 1: coded payload of the tensor's codec family; 0: raw plane bytes
  uint32_t lut;    // LDS table slot of a coded plane
};

// Codec family of a fused tensor: which GPU-native codec its coded planes use.
enum IlvFamily : uint32_t {
  kFamilyHuff = 0,  // huff_ilv (this file)
  kFamilyRans = 1,  // rans_ilv (rans_ilv.h)
};

struct IlvTensor {
  uint64_t out;    // output tensor address (16-byte aligned)
  uint64_t n;      // plane length (elements)
  uint32_t chain;
  uint32_t n_planes;
  IlvPlane planes[4];
  uint32_t family;  // IlvFamily
  // huff_ilv family, chains with CRC-able planes (crc_chain_supported): the
  // zero-init CRC-32 of every whole 16 KiB block of each plane, relative to
  // the block's end, goes to crc_part[4 * (crc_first + block) + plane];
  // kIlvNoCrc: none
  uint32_t crc_first;
};
constexpr uint32_t kIlvNoCrc = 0xFFFFFFFFu;
constexpr uint32_t kIlvCrcWords = 2048;  // LDS words of the fused CRC's tables (T0..T3, 1 KiB advance)

struct IlvEncPlane {
  uint64_t src;        // plane bytes (16-byte aligned)
  uint64_t n;
  uint32_t code_slot;  // index of its 256-entry code table
  uint32_t pad;
};

struct IlvEncBlock {
  uint64_t dst;        // device address of the block's data (lane counts first)
  uint32_t plane;
  uint32_t block;      // block index within the plane
  uint32_t lw;         // row of this block in the size pass's lane word counts
  uint32_t pad;
};

// Packed-nibble payload (tag 2): [2][n u32][0 0 0][ceil(n / 2) bytes].
constexpr uint32_t kPackedHeadBytes = 8;

// A packed-nibble payload body (tag 2): n symbols < 16 at src (16-byte
// aligned) packed two per byte to dst (8-byte aligned).
struct IlvPackJob {
  uint64_t src;
  uint64_t dst;
  uint64_t n;
};

// Launch chain code of the two-chain decode kernel: tensors of chains `a`
// and `b` (huff_ilv family, no fused CRC) in one launch, e.g. MXFP4 weights
// (nibble split) with their E8M0 scales (passthrough).
constexpr uint32_t ilv_chain_pair(uint32_t a, uint32_t b) { return 0x100u | a << 4 | b; }
constexpr bool ilv_is_pair(uint32_t code) { return code >= 0x100u; }
constexpr uint32_t ilv_pair_a(uint32_t code) { return (code >> 4) & 15u; }
constexpr uint32_t ilv_pair_b(uint32_t code) { return code & 15u; }
constexpr uint32_t kIlvPairNibblePass = ilv_chain_pair(5, 6);
// whether a tensor of chain `chain` belongs to a launch of chain code `code`
constexpr bool ilv_code_has(uint32_t code, uint32_t chain) {
  return ilv_is_pair(code) ? (chain == ilv_pair_a(code) || chain == ilv_pair_b(code)) : chain == code;
}

// A launch of at most kIlvInlineTensors tensors carries their descriptors
// in its kernel arguments (no upload before it): tensor j of the launch is
// t[j], its status word status[tix[j]], its tiles tpre[j] .. tpre[j+1] - 1.
constexpr uint32_t kIlvInlineTensors = 4;
struct IlvInline {
  uint32_t m;  // 0: the descriptors are in device memory (the pointer arguments)
  uint32_t tpre[kIlvInlineTensors + 1];
  uint32_t tix[kIlvInlineTensors];
  uint32_t pad[2];
  IlvTensor t[kIlvInlineTensors];
};

// Fused decode of the tensors tix[0..m) (indexes into `tensors`, all of
// chain `chain`); tensor tix[j] owns the 4-block tiles tpre[j] ..
// tpre[j+1] - 1 (or the same from `inl` when inl.m is nonzero).  grid:
// persistent workgroups, each taking an equal range of tiles.  n_slots: LDS
// table slots per workgroup (>= the coded planes of any tensor);
// stage_words: LDS staging words per wavefront (multiple of 4); blocks
// needing more are decoded from global memory.  status: one word per tensor
// index, zero before the launch, in host-coherent memory (the kernel ORs
// its error bits in at system scope).  crc_tab: the CRC tables
// (crc_device.h layout) when some tensor has crc_first set, else null; the
// kernel then also writes the CRC block partials to crc_part.
hipError_t launch_ilv_decode(uint32_t chain, const IlvTensor* tensors, const uint32_t* tix, const uint32_t* tpre,
                             uint32_t m, const IlvInline& inl, uint32_t grid, uint32_t* status, uint32_t n_slots,
                             uint32_t stage_words, const uint32_t* crc_tab, uint32_t* crc_part, hipStream_t stream);
size_t ilv_decode_lds_bytes(uint32_t chain, uint32_t n_slots, uint32_t stage_words, bool crc);
hipError_t ilv_decode_occupancy(uint32_t chain, uint32_t n_slots, uint32_t stage_words, bool crc, int* wg_per_cu);
hipError_t launch_ilv_pack(const IlvPackJob* jobs, uint32_t n_jobs, uint64_t max_n, hipStream_t stream);

// Stored and Identity payload bodies: n plane bytes from src to dst + shift;
// shift 1 (stored form) also writes the tag byte 0 at dst.
struct IlvStoreJob {
  uint64_t src;  // 16-byte aligned
  uint64_t dst;
  uint64_t n;
  uint32_t shift;  // 0 or 1
  uint32_t pad;
};
hipError_t launch_ilv_store(const IlvStoreJob* jobs, uint32_t n_jobs, uint64_t max_n, hipStream_t stream);
// copies of n bytes from any source alignment to 16-byte aligned dst (shift unused)
hipError_t launch_ilv_realign(const IlvStoreJob* jobs, uint32_t n_jobs, uint64_t max_n, hipStream_t stream);
hipError_t launch_ilv_hist(const IlvEncPlane* planes, uint32_t n_planes, uint64_t max_n, uint32_t* hist,
                           hipStream_t stream);
hipError_t launch_ilv_size(const IlvEncPlane* planes, const IlvEncBlock* blocks, uint32_t n_blocks,
                           const uint32_t* codes, uint8_t* lane_words, uint32_t* block_bytes, hipStream_t stream);
// stage_words (<= kIlvEncStageMax): LDS words per workgroup for assembling
// a block's coded words (blocks with more are written lane by lane)
constexpr uint32_t kIlvEncStageMax = 4096;
hipError_t launch_ilv_encode(const IlvEncPlane* planes, const IlvEncBlock* blocks, uint32_t n_blocks,
                             const uint32_t* codes, const uint8_t* lane_words, uint32_t stage_words,
                             hipStream_t stream);

}  // namespace ptwm
