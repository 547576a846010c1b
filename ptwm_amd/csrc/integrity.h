// integrity.h -- CRC-32 of decoded planes and XXH64 of restored tensors on the GPU.
#pragma once

#include <vector>

#include "runtime.h"

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

struct HashTask {  // XXH64 (seed 0) of n bytes at src (16-byte aligned)
  uint64_t src;
  uint64_t n;
};

bool crc_chain_supported(uint32_t chain);

// CRC-32/ISO-HDLC of every plane of every task, in task order (planes of a
// task consecutive).  Blocks until done.
int64_t crc32_planes(DevCtx& ctx, const std::vector<CrcTask>& tasks, std::vector<uint32_t>& crcs);

// XXH64 with seed 0 of every task's bytes.  Blocks until done.
int64_t xxh64_buffers(DevCtx& ctx, const std::vector<HashTask>& tasks, std::vector<uint64_t>& hashes);

}  // namespace ptwm
