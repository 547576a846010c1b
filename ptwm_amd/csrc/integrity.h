// integrity.h -- CRC-32 of decoded planes (GPU) and XXH64 of restored
// tensors (host cores, fed by device-to-host copies).
#pragma once

#include <vector>

#include "runtime.h"
#include "xxh64_host.h"

namespace ptwm {

struct CrcRange {  // a run of whole elements: src = first element's address, n = plane bytes
  uint64_t src;
  uint64_t n;
};
struct CrcPlane {  // one plane's CRC: its ranges and which plane of the chain
  uint64_t n;
  uint32_t range_len, first_range, n_ranges, plane;
};
static_assert(sizeof(CrcPlane) == 24, "CrcPlane layout");

// One buffer to checksum: `n` elements at `src` (16-byte aligned).  chain =
// kChainPassthrough: the buffer is one plane; kChainIeee16Split2 /
// kChainIeee32Split4: a restored tensor, CRC of each of its planes.
struct CrcTask {
  uint64_t src;
  uint64_t n;
  uint32_t chain;
};

struct HashTask {  // XXH64 (seed 0) of n device bytes at src (any alignment)
  uint64_t src;
  uint64_t n;
};


bool crc_chain_supported(uint32_t chain);

// CRC-32/ISO-HDLC of every plane of every task, in task order (planes of a
// task consecutive).  Blocks until done.
int64_t crc32_planes(DevCtx& ctx, const std::vector<CrcTask>& tasks, std::vector<uint32_t>& crcs);

// The CRC tables (crc_device.h layout) on the device, built and uploaded
// once per device.
int64_t crc_tables(DevCtx& ctx, const uint32_t** tab);

// CRC of planes whose ranges' zero-init partial CRCs (relative to each
// range's end) are on the device at d_part[4 * range + plane], e.g. the
// block partials of the fused decode.  Blocks until done.
int64_t crc32_combine(DevCtx& ctx, const std::vector<CrcPlane>& planes, const uint32_t* d_part,
                      std::vector<uint32_t>& crcs);

// A tensor decoded by the fused huff_ilv kernel with CRC partials: the
// zero-init CRC of each whole kFusedCrcBlock-byte block of each plane,
// relative to the block's end, at part[4 * (first_block + block) + plane].
constexpr uint32_t kFusedCrcBlock = 16384;
struct FusedCrc {
  uint64_t out;  // restored tensor (16-byte aligned)
  uint64_t n;    // plane length
  uint32_t chain;
  uint32_t first_block;
};

// CRC-32/ISO-HDLC of every plane of every tensor (planes of a tensor
// consecutive): the partial last blocks from the restored tensors, then the
// block partials combined.  Blocks until done.
int64_t crc32_fused(DevCtx& ctx, const std::vector<FusedCrc>& tensors, uint32_t* d_part, std::vector<uint32_t>& crcs);

// XXH64 with seed 0 of every task's bytes, after the work queued on
// ctx.stream: the buffers are copied to pinned host memory in chunks by up to
// kHashWorkers threads and hashed there.  Blocks until done.
int64_t xxh64_buffers(DevCtx& ctx, const std::vector<HashTask>& tasks, std::vector<uint64_t>& hashes);

}  // namespace ptwm
