// decode_sync.h -- parallel decode of the reference's Huffman streams.
#pragma once

#include "runtime.h"

namespace ptwm {

// Bits per subsequence: one lane decodes one subsequence of a stream.  A
// multiple of 32 with an odd word count, so lanes of a wavefront start in
// different LDS banks: 480 unless a launch has too few wavefronts to fill
// the device, then down to 96 (chosen per payload by the host).
constexpr uint32_t kSyncSubBitsMax = 480, kSyncSubBitsMin = 96;
// Payloads (Huffman, tag 1) at least this long take the parallel path.
constexpr uint64_t kSyncMinBytes = 16384;

// One of the four streams of a deferred payload, written by the exact
// kernel once the header and the decode table are known.
struct SyncStream {
  uint64_t src;        // device address of stream byte 0
  uint64_t m;          // stream bytes
  uint64_t dst;        // device address of the segment's first output byte
  uint64_t n;          // symbols of the segment (split_four of orig_len)
  uint32_t sub_bits;   // bits per subsequence
  uint32_t reserved;
  uint32_t job;        // index into the job / status arrays
  uint32_t first_sub;  // global slot of the stream's subsequence 0
  uint32_t n_sub;      // ceil(8 m / sub_bits)
  uint16_t max_bits;   // decode table width
  uint16_t fixed_len;  // every code max_bits long (a fixed-length code): max_bits, else 0
  uint32_t table;      // deferred payload slot (decode table index)
  uint32_t pad;
};
static_assert(sizeof(SyncStream) == 64, "SyncStream layout");

// Decode the jobs hj[0..n) (host copies; uploaded here).  Reference-format
// Huffman payloads of at least kSyncMinBytes decode on the parallel path;
// a payload it declines, and every other job, decode on the exact path.
// On return (stream synchronised) the host status array ctx.h_status holds
// each job's final status.
int64_t decode_jobs(DevCtx& ctx, DecodeJob* hj, size_t n_jobs);

// The same in two phases, so that a caller can queue work that reads the
// decoded planes (the merge) before it waits: decode_jobs_launch queues
// every kernel and the copy of the statuses to ctx.h_status; after the
// caller has synchronised the stream, decode_jobs_complete re-runs what the
// parallel path did not settle or declined (launching and waiting as
// needed) and reports in `rewritten` whether any job's output was written
// again after the launch phase.  The device arguments of the launch live in
// ExactRun until the next call on the device.
struct SyncArrays {
  uint64_t* start;        // per subsequence: first bit (stream-absolute)
  uint64_t* exit;         // first codeword boundary at or past the subsequence end
  uint32_t* count;        // symbols decoded from start to exit
  uint32_t* wave_sum;     // per launched wavefront: symbols of its 64 subsequences
  uint64_t* wave_prefix;  // per launched wavefront: symbols of the stream before it
  uint32_t* verdict;      // per deferred payload: its streams' verdict bits
  uint64_t* pub;          // per launched wavefront: look-back slot, (epoch << 8) | last exit past the span
  uint64_t epoch;         // this launch's look-back tag
  uint32_t look_back;     // 0: the first pass does not look back (a test mode)
};
struct ExactRun {
  const DecodeJob* jobs = nullptr;
  uint32_t* status = nullptr;
  SyncStream* streams = nullptr;
  uint16_t* tables = nullptr;
  SyncArrays A{};
  const uint32_t* wave_job = nullptr;
  const uint32_t* job_wave0 = nullptr;
  uint32_t nw = 0, n_def = 0;
  uint32_t out_stage = 16384;  // LDS output staging of the write pass, bytes per wavefront
};
int64_t decode_jobs_launch(DevCtx& ctx, DecodeJob* hj, size_t n_jobs, ExactRun& run);
int64_t decode_jobs_complete(DevCtx& ctx, DecodeJob* hj, size_t n_jobs, ExactRun& run, bool& rewritten);

// Stored (tag 0 / Identity) payloads at least this long are copied by a
// multi-workgroup kernel after the exact kernel has parsed them.
constexpr uint64_t kCopyDeferMin = 4096;
// Output bytes per workgroup of that copy: small payloads in small pieces
// (enough workgroups to fill the device), large ones in 64 KiB pieces.
__host__ __device__ inline uint64_t copy_chunk(uint64_t len) { return len >= (8ull << 20) ? 65536ull : 8192ull; }
// Fix passes queued after the first pass of the parallel Huffman decode
// (the first pass's look-back leaves them little to do).
constexpr uint32_t kFixQueued = 1;

// exact-path kernel launch (decode_exact.hip); copy_src (may be null): per
// job, the source of a deferred stored-bytes copy (0: none)
// Decode tables of the parallel path: a slot of 2048 16-bit entries per
// payload, (code length << 8) | symbol, indexed by the next max_bits stream
// bits (first bit lowest).
constexpr uint32_t kSyncTableEntries = 2048;
hipError_t launch_decode_exact(const DecodeJob* jobs_dev, uint32_t* status_dev, uint32_t n_jobs,
                               SyncStream* sync_streams, uint16_t* sync_tables, uint64_t* copy_src,
                               hipStream_t stream);
// tANS chains of the jobs with codec tANS (launch_decode_exact parses them
// too and reports their refusals, stored payloads and empty planes).
hipError_t launch_tans_decode(const DecodeJob* jobs_dev, uint32_t* status_dev, uint32_t n_jobs, hipStream_t stream);
// Zstd payloads of the job list (zstd_device.hip): one workgroup per job,
// jobs of other codecs are left to the exact kernel
hipError_t launch_zstd_decode(const DecodeJob* jobs_dev, uint32_t* status_dev, uint32_t n_jobs, hipStream_t stream);
// Order1ScaleAC payloads of the job list (o1sac_device.hip): one wavefront
// per job, jobs of other codecs are left to the other kernels.  A job's
// state: its chunk frame's, else pad[0..1] = state address, pad[2] = state
// length | format version << 24; pad[3] = the plane's row length (0 Flat).
// The reference rANS jobs of the list (decode_exact.hip; the other codecs'
// jobs are launch_decode_exact's).
hipError_t launch_rans_exact(const DecodeJob* jobs_dev, uint32_t* status_dev, uint32_t n_jobs, uint64_t* copy_src,
                             hipStream_t stream);
hipError_t launch_o1sac_decode(const DecodeJob* jobs_dev, uint32_t* status_dev, uint32_t n_jobs, hipStream_t stream);

}  // namespace ptwm
