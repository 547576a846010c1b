// dtype_codes.h -- the reference's public dtype codes as the container
// layouts use them (host code, shared by the reader and the writers).
#pragma once

#include <cstdint>
#include <vector>

namespace ptwm {

inline int chain_dtype_for_public(uint16_t code) {  // source.rs:69-88
  switch (code) {
    case 1: case 2: return 0x0003;
    case 4: case 5: return 0x0002;
    case 6: return 0x000F;
    case 13: return 0x0006;
    case 15: return 0x000A;
    case 17: return 0x0005;
    case 18: case 19: return 0x0007;
    case 20: case 21: return 0x0009;
    case 22: case 23: return 0x000B;
    case 29: return 0x0010;
    case 30: return 0x0011;
    case 31: return 0x001F;
    default: return -1;
  }
}

// public dtype codes (dtype.rs:79-103): element size, 0 = unknown
inline int public_elem_size(uint16_t code) {
  switch (code) {
    case 13: case 17: case 24: case 29: case 30: case 31: return 1;
    case 4: case 5: case 6: case 18: case 19: return 2;
    case 1: case 2: case 15: case 20: case 21: return 4;
    case 22: case 23: return 8;
    default: return 0;
  }
}
inline const char* canonical_name(uint16_t code) {  // dtype.rs:131-152
  switch (code) {
    case 1: return "float32";
    case 2: return "float";
    case 4: return "float16";
    case 5: return "half";
    case 6: return "bfloat16";
    case 13: return "uint8";
    case 15: return "uint32";
    case 17: return "int8";
    case 18: return "int16";
    case 19: return "short";
    case 20: return "int32";
    case 21: return "int";
    case 22: return "int64";
    case 23: return "long";
    case 24: return "bool";
    case 29: return "float8_e4m3fn";
    case 30: return "float8_e5m2";
    case 31: return "float4_e2m1fn_x2";
    default: return nullptr;
  }
}

// bound_source_params (source.rs:95-109): u8 ndim, u32 dims, u16 chain dtype
inline bool bound_source_params(const std::vector<uint64_t>& shape, uint16_t dtype, std::vector<uint8_t>& out) {
  const int cd = chain_dtype_for_public(dtype);
  if (cd < 0 || shape.size() > 255) return false;
  out.clear();
  out.push_back((uint8_t)shape.size());
  for (uint64_t d : shape) {
    if (d > 0xFFFFFFFFull) return false;
    for (int k = 0; k < 4; ++k) out.push_back((uint8_t)(d >> (8 * k)));
  }
  out.push_back((uint8_t)cd);
  out.push_back((uint8_t)(cd >> 8));
  return true;
}

}  // namespace ptwm
