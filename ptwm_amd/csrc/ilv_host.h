// ilv_host.h -- host orchestration of the huff_ilv codec.
#pragma once

#include <vector>

#include "huff_ilv.h"
#include "runtime.h"

namespace ptwm {

struct IlvEncResult {
  uint64_t offset;  // payload offset inside the output buffer (256-byte aligned)
  uint64_t len;     // payload length
  uint32_t coded;   // 1: huff_ilv coded payload; 0: stored
  uint32_t codec;   // codec wire id of the payload (huff_ilv, or identity when stored as identity)
};

// Encode np planes (16-byte aligned device buffers) into out_dev.  Planes that
// do not shrink are stored: as Identity payloads when identity_fallback,
// else as huff_ilv tag-0 payloads.  Returns the bytes used, or
// kBufferTooSmall with *needed set.
int64_t ilv_encode_planes(DevCtx& ctx, const uint64_t* src, const uint64_t* n, uint32_t np, uint64_t out_dev,
                          uint64_t out_cap, bool identity_fallback, IlvEncResult* res, uint64_t* needed);

// The same for the rans_ilv codec (rans_host.hip).
int64_t rilv_encode_planes(DevCtx& ctx, const uint64_t* src, const uint64_t* n, uint32_t np, uint64_t out_dev,
                           uint64_t out_cap, bool identity_fallback, IlvEncResult* res, uint64_t* needed);

// Decode and merge the given tensors (fused path; each tensor's coded planes
// are of its codec family).  Returns kOk or kInvalidInput.
int64_t ilv_decode_tensors(DevCtx& ctx, const std::vector<IlvTensor>& tensors);

}  // namespace ptwm
