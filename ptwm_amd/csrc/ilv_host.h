// ilv_host.h -- host orchestration of the huff_ilv codec.
#pragma once

#include <vector>

#include "huff_ilv.h"
#include "runtime.h"

namespace ptwm {

struct IlvEncResult {
  uint64_t offset;  // payload offset inside the output buffer (256-byte aligned)
  uint64_t len;     // payload length
  uint32_t coded;   // 1: coded payload (tag 1); 0: stored or packed
  uint32_t codec;   // codec wire id of the payload (huff_ilv, or identity when stored as identity)
};

// Encode np planes (16-byte aligned device buffers) into out_dev.  Planes that
// do not shrink are stored: as Identity payloads when identity_fallback,
// else as huff_ilv tag-0 payloads.  Returns the bytes used, or
// kBufferTooSmall with *needed set.
int64_t ilv_encode_planes(DevCtx& ctx, const uint64_t* src, const uint64_t* n, uint32_t np, uint64_t out_dev,
                          uint64_t out_cap, bool identity_fallback, IlvEncResult* res, uint64_t* needed);

// Payload forms of both GPU-native codecs.
enum IlvForm : uint32_t { kFormStored = 0, kFormCoded = 1, kFormPacked = 2, kFormIdentity = 3 };

// True when the 256-bin histogram has no symbol >= 16.
inline bool all_nibbles(const uint32_t* hist) {
  for (int s = 16; s < 256; ++s)
    if (hist[s]) return false;
  return true;
}

// The encoders' choice of payload form (the format specification's rule):
// coded (tag 1) when strictly smaller than both other forms; else packed
// nibbles (tag 2) when every symbol is < 16 and that beats storing; else
// stored (tag 0).  With identity_fallback, a stored plane and any payload
// not smaller than n become an Identity payload of n bytes.  *len: the
// payload length of the chosen form.
uint32_t ilv_choose_form(uint64_t n, bool nibbles, bool codable, uint64_t coded_len, bool identity_fallback,
                         uint64_t* len);

// Write the stored, packed and Identity payloads among res[0..np) (form[p]
// as chosen above) on ctx.stream: tag bytes and packed headers from `keep`
// (host memory the caller keeps alive until the stream is synchronised),
// plane copies and one pack launch.  Returns kOk or an error status.
int64_t ilv_store_planes(DevCtx& ctx, const uint64_t* src, const uint64_t* n, uint32_t np, uint64_t out_dev,
                         const IlvEncResult* res, const uint32_t* form, std::vector<uint8_t>& keep);

// The same for the rans_ilv codec (rans_host.hip).
int64_t rilv_encode_planes(DevCtx& ctx, const uint64_t* src, const uint64_t* n, uint32_t np, uint64_t out_dev,
                           uint64_t out_cap, bool identity_fallback, IlvEncResult* res, uint64_t* needed);

// Decode and merge the given tensors (fused path; each tensor's coded planes
// are of its codec family).  Returns kOk or kInvalidInput.
int64_t ilv_decode_tensors(DevCtx& ctx, const std::vector<IlvTensor>& tensors, bool all_slots = false);

}  // namespace ptwm
