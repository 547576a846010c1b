// runtime.h -- per-device context, scratch memory and decode-plan execution.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "plan_types.h"
#include "ptwm_common.h"

namespace ptwm {

// Grow-only device allocation reused across calls on one device.  A
// borrowed buffer is a view of memory owned elsewhere (the allocation-free
// decode's fixed scratch): ensure() never allocates for it and fails when
// the view is too small.
struct DeviceBuffer {
  void* ptr = nullptr;
  size_t cap = 0;
  bool borrowed = false;
  hipError_t ensure(size_t bytes);
  ~DeviceBuffer();
};

struct PinnedBuffer {
  void* ptr = nullptr;
  size_t cap = 0;
  bool borrowed = false;
  unsigned flags = hipHostMallocDefault;  // hipHostMallocCoherent: kernels write it directly
  hipError_t ensure(size_t bytes);
  ~PinnedBuffer();
};

// The allocation-free decode (ptwm_mi355x_dispatch_decode_noalloc_cuda):
// all its device scratch lives in one fixed array per device (runtime.hip),
// laid out as [CRC tables][tensor descriptors, launch indexes, status]
// [CRC range arguments][CRC combine arguments][exact-route stubs][CRC block
// partials], and its host staging in a fixed per-device host area.
constexpr uint64_t kNoAllocScratchBytes = 16ull << 20;
constexpr uint64_t kNoAllocTabOff = 0, kNoAllocTabBytes = 16ull << 10;
constexpr uint64_t kNoAllocArgsOff = kNoAllocTabOff + kNoAllocTabBytes, kNoAllocArgsBytes = 1ull << 20;
constexpr uint64_t kNoAllocCrcArgsOff = kNoAllocArgsOff + kNoAllocArgsBytes, kNoAllocCrcArgsBytes = 1ull << 20;
constexpr uint64_t kNoAllocCombOff = kNoAllocCrcArgsOff + kNoAllocCrcArgsBytes, kNoAllocCombBytes = 512ull << 10;
constexpr uint64_t kNoAllocStubOff = kNoAllocCombOff + kNoAllocCombBytes, kNoAllocStubBytes = 4096;
constexpr uint64_t kNoAllocPartOff = kNoAllocStubOff + kNoAllocStubBytes;
constexpr uint64_t kNoAllocPartBytes = kNoAllocScratchBytes - kNoAllocPartOff;
constexpr uint64_t kNoAllocHostBytes = 1ull << 20;
// host-coherent status words of the fused decode (one per tensor)
constexpr uint64_t kNoAllocStatusBytes = 16ull << 10;
static_assert(kNoAllocStatusBytes >= 4ull * 4096, "a status word for every tensor the allocation-free decode takes");
// limits of a plan the allocation-free decode accepts
constexpr uint32_t kNoAllocMaxTensors = 4096;
constexpr uint64_t kNoAllocMaxCrcBlocks = kNoAllocPartBytes / 16;

// One host hashing worker (hash_host.hip): its stream, two pinned chunk
// buffers and their copy-done events.
constexpr uint64_t kHashChunk = 16ull << 20;
constexpr uint32_t kHashWorkers = 8;
struct HashWorker {
  hipStream_t stream = nullptr;
  void* pinned[2] = {nullptr, nullptr};
  hipEvent_t ev[2] = {nullptr, nullptr};
  hipError_t init();
};

// Input bytes per batch of the batched tensor encoder (its plane scratch).
constexpr uint64_t kDefaultEncBatchBytes = 4ull << 30;

// One per device ordinal.  All entry points serialise on `mu`: the stream
// and the scratch buffers are shared by every call on that device.
struct DevCtx {
  int dev = -1;
  hipStream_t stream = nullptr;      // the stream of the current call (own_stream or the caller's)
  hipStream_t own_stream = nullptr;  // the library's stream of this device
  std::mutex mu;
  DeviceBuffer jobs;     // DecodeJob array
  DeviceBuffer status;   // per-job status words
  DeviceBuffer planes;   // decoded plane scratch (unfused path)
  DeviceBuffer aux;      // small per-call tables
  PinnedBuffer h_jobs;
  PinnedBuffer h_status;
  PinnedBuffer h_small;
  // huff_ilv encoder / decoder scratch
  DeviceBuffer enc_planes, enc_hist, enc_codes, enc_blocks, enc_lane_words, enc_block_bytes, enc_pack;
  DeviceBuffer crc_comb, crc_part;  // CRC combine arguments; fused-decode CRC block partials
  DeviceBuffer ilv_args, ilv_realign, realign_jobs;
  PinnedBuffer h_realign;
  // reference-format (Huffman / rANS) encoder scratch
  DeviceBuffer ref_jobs, ref_hist, ref_segs, ref_seglen, ref_codes, ref_rans_tab, ref_rans_segs, ref_rans_scratch,
      ref_rans_len, ref_hdr, ref_pack, ref_ops;
  PinnedBuffer h_enc, h_ilv;
  // fused-decode status words, written by the kernels (host-coherent)
  PinnedBuffer h_ilv_status;
  // parallel Huffman decode of reference streams
  DeviceBuffer sync_tables, sync_sub, sync_waves, sync_pub;
  PinnedBuffer h_job_status;  // the exact route's status words, written by the kernels (host-coherent)
  uint64_t sync_epoch = 0;  // look-back tag of the parallel Huffman decode's first pass, one per launch
  DeviceBuffer exact_args;  // the exact route's argument arrays, one upload per call
  // reference Huffman payloads of the exact route, cumulative: accepted by
  // the parallel path, decoded again by the exact state machine, and calls
  // that needed fix passes beyond the queued ones
  uint64_t sync_accepted = 0, sync_fallbacks = 0, sync_extra_rounds = 0;
  PinnedBuffer h_exact_args;
  // inverse plane ops (plane_ops.hip): job list and IntDelta tile sums
  DeviceBuffer op_jobs, op_sums;
  PinnedBuffer h_op;
  // chunk frame headers of GPU-native planes (gathered before the decode)
  DeviceBuffer chunk_addr, chunk_head;
  PinnedBuffer h_chunk;
  // integrity (CRC-32 / XXH64) tables and arguments
  DeviceBuffer crc_tab, crc_args;
  std::vector<HashWorker> hash_workers;  // XXH64 on host cores (hash_host.hip)
  hipEvent_t hash_ready = nullptr;       // the restore is complete before the copies
  bool crc_tab_ready = false;
  int cu_count = 0;  // compute units of the device (0: not queried yet)
  std::map<uint64_t, int> ilv_occupancy;  // (chain, slots, stage words) -> workgroups per CU
  DeviceBuffer stage_in, stage_out, enc_split;
  uint64_t enc_batch_bytes = kDefaultEncBatchBytes;  // ptwm_mi355x_set_encode_batch_bytes
  // optional per-phase kernel timing with HIP events on `stream`
  bool profile = false;
  hipEvent_t ev[4] = {nullptr, nullptr, nullptr, nullptr};
  hipEvent_t order_ev = nullptr;  // producer-stream ordering (ptwm_mi355x_stream_wait)
  // the exact route's reference rANS jobs run on a second stream, beside
  // its Huffman kernels (forked from and joined back to `stream`)
  hipStream_t side_stream = nullptr;
  hipEvent_t side_fork = nullptr, side_join = nullptr;
  hipError_t ensure_side();
  float last_ms[3] = {0, 0, 0};  // entropy decode, merge, whole call
  hipError_t ensure_events();
  // allocation-free decode: this device's copy of the fixed scratch array
  // (its device address, resolved once at set-up; null if that failed), the
  // host staging area (allocated at set-up) and whether the CRC tables are
  // in the scratch yet
  uint8_t* noalloc_dev = nullptr;
  std::unique_ptr<uint8_t[]> noalloc_host;
  void* noalloc_status = nullptr;  // kNoAllocStatusBytes of host-coherent memory
  bool noalloc_tab_ready = false;
};

// Returns nullptr if the ordinal is invalid or HIP initialisation fails.
// Creates the device's context on its first call (a stream, pinned status
// words, the allocation-free decode's scratch address).
DevCtx* get_ctx(uint32_t device_ordinal);
// The device's context if it exists, else nullptr; never creates one.
DevCtx* find_ctx(uint32_t device_ordinal);

// Process-wide count of the library's own hipMalloc / hipHostMalloc calls
// and stream / event creations (ptwm_mi355x_alloc_calls); every such call
// site counts itself with note_alloc().
void note_alloc();
uint64_t alloc_calls();


// Decode every tensor of the plan from in_dev into out_dev (device
// addresses).  Blocks until the work has completed.  Returns kOk or an
// error code.
int64_t execute_plan(DevCtx& ctx, const Plan& plan, uint64_t in_dev, uint64_t out_dev);

// The same without allocating device or pinned memory: every tensor must
// take the fused route (fused_eligible), carry no XXH64, have 4-byte aligned
// coded payloads and fit the fixed scratch (kNoAllocMaxTensors,
// kNoAllocMaxCrcBlocks); kUnsupported otherwise, kMissingCapability when the
// device's scratch address could not be resolved.
int64_t execute_plan_noalloc(DevCtx& ctx, const Plan& plan, uint64_t in_dev, uint64_t out_dev);

// Whether the tensor is restored by the fused decode kernel (every plane an
// unchunked GPU-native payload of one codec family or a stored Identity
// plane, at least one coded, 16-byte aligned output, and a plane CRC only
// for the chains the fused CRC covers).
bool fused_eligible(const PlanTensor& T, uint64_t out_dev);

// kernel launchers (transform.hip; the decode launchers are in decode_sync.h)
hipError_t launch_merge(uint32_t chain, const uint8_t* const* planes, uint64_t plane_len, uint8_t* out,
                        hipStream_t stream);
hipError_t launch_split(uint32_t chain, const uint8_t* in, uint64_t plane_len, uint8_t* const* planes,
                        hipStream_t stream);
hipError_t launch_copy(const uint8_t* in, uint8_t* out, uint64_t n, hipStream_t stream);


}  // namespace ptwm
