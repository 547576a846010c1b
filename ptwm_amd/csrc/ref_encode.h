// ref_encode.h -- GPU encoder of the reference's Huffman / rANS plane
// payloads (byte-identical to the reference encoder; see ref_encode.hip).
#pragma once

#include <vector>

#include "ptwm_common.h"
#include "runtime.h"

namespace ptwm {

struct RefJobDev {
  uint64_t src;
  uint64_t n;
};

// One of the four split_four segments of a coded job.
struct RefSegDev {
  uint64_t src;           // first symbol
  uint64_t n;             // symbols
  uint64_t words;         // Huffman: 32-bit words of its packed stream
  uint64_t scratch_word;  // Huffman: first word of its area in the pack scratch
  uint64_t scratch_byte;  // rANS: its area in the rANS scratch
  uint32_t table;         // job index (code / frequency tables)
  uint32_t pad;
};

// A slice of a Huffman segment packed by one workgroup: symbols
// [sym0, sym0 + n) of segment seg.
struct RefSliceDev {
  uint64_t sym0;
  uint64_t n;
  uint32_t seg;
  uint32_t pad[3];
};
constexpr uint64_t kSliceSyms = 1ull << 15;

struct RefCopyOp {
  uint64_t src, dst, n;
  uint64_t rev_from;  // bytes from here on are copied from the source's end backward
};

// A payload to encode: n bytes at device address src with codec kCodecHuffman
// or kCodecRans.
struct RefJob {
  uint64_t src;
  uint64_t n;
  uint32_t codec;
};

// Two phases so that callers can lay out frames before anything is written:
// plan() computes every payload's exact size (running the histogram, table,
// size and rANS passes), write() then places each payload at its device
// address.  Both run on the context's stream and synchronise it.
class RefEncoder {
 public:
  int64_t plan(DevCtx& ctx, const std::vector<RefJob>& jobs, std::vector<uint64_t>& payload_len);
  // literal: (device address, bytes) written as well (chunk frame headers);
  // copies: further device-to-device copies (Identity planes and chunks)
  int64_t write(DevCtx& ctx, const std::vector<uint64_t>& dst,
                const std::vector<std::pair<uint64_t, std::vector<uint8_t>>>& literal = {},
                const std::vector<RefCopyOp>& copies = {});

 private:
  struct JobInfo {
    bool raw = true;              // stored as [00] + bytes (or [00] when empty)
    std::vector<uint8_t> header;  // weights header / frequency header
    uint32_t seg0 = 0;            // first of its four segments
    uint64_t blob = 0;
  };
  std::vector<RefJob> jobs_;
  std::vector<JobInfo> info_;
  std::vector<RefSegDev> segs_;
  std::vector<uint64_t> seg_len_;   // bytes of each segment's stream
  std::vector<uint32_t> huf_codes_;  // per job 256 x (len << 16 | rev code)
  std::vector<uint32_t> rans_tab_;   // per job 256 x 4 words
  uint64_t pack_words_ = 0;
};

}  // namespace ptwm
