// plan_types.h -- the parsed decode plan (plain C++, no device types).
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "codes.h"

namespace ptwm {

// Parsed decode plan (the state bytes of the hardware-backend entry point).
struct PlanChunk {
  uint32_t offset_in_payload;
  uint32_t decoded_size;
};
struct PlanPlane {
  uint32_t codec = 0;
  bool chunked = false;
  uint64_t payload_offset = 0;
  uint64_t payload_len = 0;
  uint64_t plane_len = 0;
  uint32_t crc32 = 0;
  uint32_t op = kPlaneOpNone;  // inverse plane op after the decode (codes.h)
  uint32_t op_param = 0;       // its element width in bytes, or k
  // codec state and plane layout (Order1ScaleAC): the state bytes at
  // [state_offset, +state_len) of the input (chunked planes: each chunk
  // frame's own), its format version, and the row length (0 = Flat)
  bool has_state = false;
  uint64_t state_offset = 0;
  uint32_t state_len = 0, row_len = 0, state_version = 0;
  std::vector<PlanChunk> chunks;
};
struct PlanTensor {
  uint64_t out_offset = 0;
  uint64_t out_len = 0;
  uint32_t chain = 0;
  bool has_crc = false;
  bool has_hash = false;  // xxh64 (seed 0) of the restored tensor
  uint64_t xxh64 = 0;
  std::vector<PlanPlane> planes;
};
struct Plan {
  std::vector<PlanTensor> tensors;
};

// Parse + validate against the input/output buffer sizes.  Returns kOk or
// kInvalidInput.
int64_t parse_plan(const uint8_t* state, size_t state_len, uint64_t in_len, uint64_t out_len, Plan& plan);

// planes per chain and tensor bytes per plane element (fusion.rs)
int chain_planes(uint32_t chain);
int chain_ratio(uint32_t chain);

}  // namespace ptwm
