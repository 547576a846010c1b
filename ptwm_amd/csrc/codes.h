// codes.h -- return codes, codec wire ids and chain kinds (plain C++).
//
// Return codes follow the reference native ABI (crates/ptwm-core/src/flavor/
// native.rs:634-657): >= 0 bytes written, -1 InvalidInput, -2
// BufferTooSmall, -3 MissingCapability, -4 MissingNativeDep, -5
// Unsupported, anything else InternalError.
#pragma once

#include <cstdint>

namespace ptwm {

constexpr int64_t kOk = 0;
constexpr int64_t kInvalidInput = -1;
constexpr int64_t kBufferTooSmall = -2;
constexpr int64_t kMissingCapability = -3;
constexpr int64_t kMissingNativeDep = -4;
constexpr int64_t kUnsupported = -5;
constexpr int64_t kInternal = -6;

// Codec wire ids (crates/ptwm-core/src/codec.rs:3-23) plus this library's
// GPU-native codec, registered as a third-party plane codec.
constexpr uint32_t kCodecIdentity = 0x0000;
constexpr uint32_t kCodecHuffman = 0x0001;
constexpr uint32_t kCodecRans = 0x0003;
constexpr uint32_t kCodecZstd = 0x0004;   // RFC 8878 frames (zstd_device.hip)
constexpr uint32_t kCodecTans = 0x0007;   // entropy/tans (single stream, decode only)
constexpr uint32_t kCodecO1sac = 0x0011;  // Order1ScaleAC (range coder, stateful, decode only)
constexpr uint32_t kCodecHuffIlv = 0x7F01;  // GPU-native interleaved Huffman
constexpr uint32_t kCodecRansIlv = 0x7F02;  // GPU-native interleaved rANS

// Inverse plane ops on one terminal plane (chain/dispatch.rs:96-122; OpId
// wire ids 0x0052, 0x0053, 0x0064 of transforms/op.rs).  Parameter: the
// element width in bytes (IntDelta, PredictorXor) or k (MantissaZeroStrip).
constexpr uint32_t kPlaneOpNone = 0;
constexpr uint32_t kPlaneOpIntDelta = 1;
constexpr uint32_t kPlaneOpPredictorXor = 2;
constexpr uint32_t kPlaneOpMantissaZeroStrip = 3;

// Chain kinds: the fused reorder+split pairs of transforms/fusion.rs plus
// the unfused NibbleSplit and BytePassthrough used by the u8 chains.
enum ChainKind : uint32_t {
  kChainIeee16Split2 = 1,
  kChainIeee32Split4 = 2,
  kChainE4m3Nibble = 3,
  kChainE5m2Nibble = 4,
  kChainNibbleSplit = 5,
  kChainPassthrough = 6,
};

}  // namespace ptwm
