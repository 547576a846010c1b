// plan_parse.cpp -- decode-plan (PTMD v1) parsing and validation.
//
// Host-only C++ with no device dependency, so that the parser of the
// untrusted state bytes also builds on its own under the sanitizers and the
// fuzzer (tests/fuzz).  Layout: include/ptwm_mi355x.h (decode plan); the
// chunk tables are the reference's (plane_record.rs:16-20).
#include <cstring>

#include "plan_types.h"

namespace ptwm {

int chain_planes(uint32_t chain) {
  switch (chain) {
    case kChainIeee16Split2: return 2;
    case kChainIeee32Split4: return 4;
    case kChainE4m3Nibble:
    case kChainE5m2Nibble:
    case kChainNibbleSplit: return 2;
    case kChainPassthrough: return 1;
    default: return -1;
  }
}

int chain_ratio(uint32_t chain) {
  switch (chain) {
    case kChainIeee16Split2: return 2;
    case kChainIeee32Split4: return 4;
    default: return 1;
  }
}

namespace {

struct Cursor {
  const uint8_t* p;
  size_t n;
  size_t off = 0;
  bool ok = true;
  template <typename T>
  T get() {
    T v{};
    if (!ok || n - off < sizeof(T)) {
      ok = false;
      return v;
    }
    std::memcpy(&v, p + off, sizeof(T));
    off += sizeof(T);
    return v;
  }
};

constexpr uint32_t kPlanMagic = 0x444D5450u;  // "PTMD"

}  // namespace

int64_t parse_plan(const uint8_t* state, size_t state_len, uint64_t in_len, uint64_t out_len, Plan& plan) {
  if (!state) return kInvalidInput;
  Cursor c{state, state_len};
  if (c.get<uint32_t>() != kPlanMagic || !c.ok) return kInvalidInput;
  uint16_t ver = c.get<uint16_t>();
  uint16_t flags = c.get<uint16_t>();
  uint32_t n_tensors = c.get<uint32_t>();
  if (!c.ok || ver != 1 || flags != 0) return kInvalidInput;
  if (n_tensors > (1u << 24)) return kInvalidInput;
  plan.tensors.resize(n_tensors);
  for (uint32_t t = 0; t < n_tensors; ++t) {
    PlanTensor& T = plan.tensors[t];
    T.out_offset = c.get<uint64_t>();
    T.out_len = c.get<uint64_t>();
    T.chain = c.get<uint8_t>();
    uint32_t np = c.get<uint8_t>();
    uint16_t tflags = c.get<uint16_t>();
    if (!c.ok) return kInvalidInput;
    T.has_crc = (tflags & 1u) != 0;
    T.has_hash = (tflags & 2u) != 0;
    if (T.has_hash) T.xxh64 = c.get<uint64_t>();
    int want_np = chain_planes(T.chain);
    if (!c.ok || want_np < 0 || (int)np != want_np || (tflags & ~3u)) return kInvalidInput;
    if (T.out_offset > out_len || out_len - T.out_offset < T.out_len) return kInvalidInput;
    T.planes.resize(np);
    for (uint32_t p = 0; p < np; ++p) {
      PlanPlane& P = T.planes[p];
      P.codec = c.get<uint16_t>();
      uint16_t pflags = c.get<uint16_t>();
      uint32_t nch = c.get<uint32_t>();
      P.payload_offset = c.get<uint64_t>();
      P.payload_len = c.get<uint64_t>();
      P.plane_len = c.get<uint64_t>();
      P.crc32 = T.has_crc ? c.get<uint32_t>() : 0;
      // bit 6: codec state and layout follow (Order1ScaleAC)
      P.has_state = (pflags & 0x40u) != 0;
      if (P.has_state) {
        P.state_offset = c.get<uint64_t>();
        P.state_len = c.get<uint32_t>();
        P.row_len = c.get<uint32_t>();
        P.state_version = c.get<uint32_t>();
        if (!c.ok || P.state_offset > in_len || in_len - P.state_offset < P.state_len || P.state_version > 255)
          return kInvalidInput;
      }
      if (!c.ok || (pflags & ~0x7Fu)) return kInvalidInput;
      P.chunked = (pflags & 1u) != 0;
      // bits 1-2: inverse plane op; bits 3-5: log2 of its element width
      // (IntDelta, PredictorXor) or k (MantissaZeroStrip)
      P.op = (pflags >> 1) & 3u;
      const uint32_t pc = (pflags >> 3) & 7u;
      if (P.op == kPlaneOpNone) {
        if (pc) return kInvalidInput;
      } else if (P.op == kPlaneOpMantissaZeroStrip) {
        if (pc == 0) return kInvalidInput;  // mantissa_zero.rs new(): k in 1..=7
        P.op_param = pc;
      } else {
        if (pc > 3) return kInvalidInput;
        P.op_param = 1u << pc;
      }
      // the ops refuse nibble-width planes (int_delta.rs, predictor_xor.rs
      // reject_nibble; mantissa_zero.rs needs byte elements)
      if (P.op != kPlaneOpNone && (T.chain == kChainE4m3Nibble || T.chain == kChainE5m2Nibble ||
                                   T.chain == kChainNibbleSplit))
        return kInvalidInput;
      if (P.codec != kCodecIdentity && P.codec != kCodecHuffman && P.codec != kCodecRans && P.codec != kCodecZstd &&
          P.codec != kCodecTans && P.codec != kCodecHuffIlv && P.codec != kCodecRansIlv && P.codec != kCodecO1sac)
        return kUnsupported;
      // Order1ScaleAC needs its state and layout; the other codecs take none
      if (P.has_state != (P.codec == kCodecO1sac)) return kInvalidInput;
      if (P.payload_offset > in_len || in_len - P.payload_offset < P.payload_len) return kInvalidInput;
      if (P.chunked) {
        if (nch == 0 || nch > (1u << 26) || state_len - c.off < (size_t)nch * 8) return kInvalidInput;
        P.chunks.resize(nch);
        uint64_t tot = 0;
        for (uint32_t k = 0; k < nch; ++k) {
          P.chunks[k].offset_in_payload = c.get<uint32_t>();
          P.chunks[k].decoded_size = c.get<uint32_t>();
          tot += P.chunks[k].decoded_size;
          // container.rs:2000-2015: offsets must not decrease and stay in the payload
          uint64_t start = P.chunks[k].offset_in_payload;
          if (start > P.payload_len) return kInvalidInput;
          if (k > 0 && start < P.chunks[k - 1].offset_in_payload) return kInvalidInput;
        }
        if (!c.ok || tot != P.plane_len) return kInvalidInput;
      } else if (nch != 0) {
        return kInvalidInput;
      }
      // every plane of a chain has the same length (fusion.rs inverse checks)
      if (P.plane_len != T.planes[0].plane_len) return kInvalidInput;
      // a delta op's plane holds whole elements (int_delta.rs:104-110)
      if ((P.op == kPlaneOpIntDelta || P.op == kPlaneOpPredictorXor) && P.plane_len % P.op_param) return kInvalidInput;
    }
    uint64_t pl = T.planes[0].plane_len;
    if (pl > T.out_len || pl * (uint64_t)chain_ratio(T.chain) != T.out_len) return kInvalidInput;
  }
  if (c.off != state_len) return kInvalidInput;
  return kOk;
}

}  // namespace ptwm
