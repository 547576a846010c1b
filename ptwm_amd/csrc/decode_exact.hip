// decode_exact.hip -- reference-format plane payload decode on gfx950.
//
// One 64-lane wavefront per independently coded unit (a plane payload or
// one chunk of a chunked plane).  The whole wave parses the payload header
// and builds the decode table in LDS; then four lanes, one per segment of
// the reference's 4-segment frame (entropy/stream_frame.rs:27-39), run the
// reference reader state machine bit for bit:
//   Huffman: entropy/huffman/decompress.rs:8-211 with the backward
//            BitReader of entropy/huffman/bitstream.rs:58-187, including the
//            lockstep 4-stream fast loop whose exit depends on all four
//            streams and the wrapping u8 bit counter, so acceptance and
//            output match the reference for every input, malformed or not.
//   rANS:    entropy/rans/decompress.rs:24-166.
// Payload framing follows codecs/huffman.rs:90-141, codecs/rans.rs:97-170,
// codec_tagged.rs:98-194 and codecs/length_prefix.rs:30-33; chunk frames
// follow container.rs:2010-2049.
//
// This kernel is the exact path: it is used for the reference formats.  A
// large Huffman payload (DecodeJob::sync_id != 0) stops after the header and
// decode table: its four streams continue on the parallel path
// (decode_sync.hip), which hands back any payload it cannot prove it decodes
// exactly as this kernel would.
// The throughput-oriented path is the huff_ilv codec (huff_ilv.hip).
#include "decode_sync.h"
#include "ptwm_common.h"

namespace ptwm {

namespace {

constexpr int kHufMaxBits = 11;
constexpr uint32_t kHdrStage = 160;  // staged Huffman header bytes: weights (<= 130) + jump table (16)
constexpr uint32_t kRansProbBits = 11;
constexpr uint32_t kRansScale = 1u << kRansProbBits;
constexpr uint32_t kRansL = 1u << 23;
// rANS stream bytes reach the four chains through one LDS ring per chain:
// kRansRing bytes (a power of two) plus a copy of its first granule after
// its end, so that the byte after the ring's last one is read at the next
// address.  Each round the wavefront stages up to kRansStageGranules
// 16-byte granules per chain (global loads issued before the round's decode
// and written to the rings after it) and every chain decodes up to
// kRansRound symbols from what is staged.
constexpr uint32_t kRansRing = 2048;
constexpr uint32_t kRansRingPad = 16;
constexpr uint32_t kRansStageGranules = 32;   // 2 per lane: 512 bytes per chain per round
constexpr uint32_t kRansRound = 256;          // <= 2 bytes per symbol: 512 bytes per chain
constexpr uint32_t kTansStageWords = 1024;    // tANS stream words staged at a time (4 KiB)

// inclusive sum over the wavefront: within each row of 16 lanes by row
// shifts, then each row's predecessors' totals through the row broadcasts
// of lanes 15 and 31
__device__ __forceinline__ uint32_t wave_incl_sum_u32(uint32_t v) {
  uint32_t x = v;
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xF, 0xF, false);  // row_shr:2
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xF, 0xF, false);  // row_shr:4
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xF, 0xF, false);  // row_shr:8
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xA, 0xF, false);  // row_bcast:15 -> rows 1, 3
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xC, 0xF, false);  // row_bcast:31 -> rows 2, 3
  return x;
}
__device__ __forceinline__ uint32_t wave_excl_sum_u32(uint32_t v) { return wave_incl_sum_u32(v) - v; }
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
  return __builtin_amdgcn_readlane(wave_incl_sum_u32(v), 63);
}

__device__ inline uint32_t ld_u32le(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// Backward bit reader, state identical to bitstream.rs:58-67.
struct Reader {
  const uint8_t* data;
  int64_t bi;       // next byte to read, moving toward 0
  uint64_t cont;    // LSB-aligned bit container
  uint32_t cnt;     // u8 in the reference; kept masked to 8 bits here
};

__device__ inline void rd_init(Reader& r, const uint8_t* d, uint64_t n) {
  r.data = d;
  r.bi = (int64_t)n - 1;
  r.cont = 0;
  r.cnt = 0;
  int64_t avail = r.bi + 1 < 8 ? r.bi + 1 : 8;   // initial_fill (bitstream.rs:76-82)
  for (int64_t i = 0; i < avail; ++i) {
    r.cont |= (uint64_t)g_ld<uint8_t>((uint64_t)(d + r.bi)) << r.cnt;
    r.cnt = (r.cnt + 8) & 0xFF;
    r.bi--;
  }
}

// reload (bitstream.rs:88-106)
__device__ inline void rd_reload(Reader& r) {
  if (r.cnt == 0 && r.bi >= 7) {
    const uint8_t* p = r.data + (r.bi - 7);
    uint64_t w = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) w = (w << 8) | g_ld<uint8_t>((uint64_t)(p + i));
    r.cont = w;
    r.cnt = 64;
    r.bi -= 8;
  } else if (r.cnt <= 32 && r.bi >= 3) {
    const uint8_t* p = r.data + (r.bi - 3);
    const uint64_t a = (uint64_t)p;
    uint32_t w = ((uint32_t)g_ld<uint8_t>(a) << 24) | ((uint32_t)g_ld<uint8_t>(a + 1) << 16) |
                 ((uint32_t)g_ld<uint8_t>(a + 2) << 8) | g_ld<uint8_t>(a + 3);
    r.cont |= (uint64_t)w << r.cnt;
    r.cnt = (r.cnt + 32) & 0xFF;
    r.bi -= 4;
  }
}

// refill (bitstream.rs:108-121)
__device__ inline void rd_refill(Reader& r) {
  if (r.cnt <= 32 && r.bi >= 3) {
    rd_reload(r);
  } else {
    while (r.cnt < 56 && r.bi >= 0) {
      r.cont |= (uint64_t)g_ld<uint8_t>((uint64_t)(r.data + r.bi)) << r.cnt;
      r.cnt = (r.cnt + 8) & 0xFF;
      r.bi--;
    }
  }
}

// decode_symbol (bitstream.rs:129-137); the counter wraps like the u8.
__device__ inline uint8_t rd_decode(Reader& r, const uint16_t* table, uint64_t mask) {
  uint16_t e = table[r.cont & mask];
  uint32_t nb = e >> 8;
  r.cont >>= nb;
  r.cnt = (r.cnt - nb) & 0xFF;
  return (uint8_t)(e & 0xFF);
}

__device__ inline void rd_refill_to(Reader& r, uint32_t nbits) {
  while (r.cnt < nbits && r.bi >= 0) {
    r.cont |= (uint64_t)g_ld<uint8_t>((uint64_t)(r.data + r.bi)) << r.cnt;
    r.cnt = (r.cnt + 8) & 0xFF;
    r.bi--;
  }
}

// decode_stream_tail (decompress.rs:152-211); returns false on error.
__device__ bool huf_tail(Reader& r, const uint16_t* table, uint64_t mask, uint32_t max_bits, uint8_t* out,
                         uint64_t len) {
  uint64_t i = 0;
  while (i < len && r.bi >= 3) {
    if (r.cnt < max_bits) rd_refill(r);
    g_st<uint8_t>((uint64_t)(out + i++), rd_decode(r, table, mask));
  }
  while (i < len) {
    uint64_t avail = (uint64_t)r.cnt + (uint64_t)(r.bi + 1 > 0 ? r.bi + 1 : 0) * 8;
    if (avail == 0) return false;
    rd_refill_to(r, max_bits);
    if (r.cnt == 0) return false;
    uint16_t e = table[r.cont & mask];
    uint32_t nb = e >> 8;
    if ((uint64_t)nb > avail) return false;
    if (nb) {
      if (r.cnt < nb) rd_refill_to(r, nb);
      if (r.cnt < nb) return false;
      r.cont >>= nb;
      r.cnt = (r.cnt - nb) & 0xFF;
    }
    g_st<uint8_t>((uint64_t)(out + i++), (uint8_t)(e & 0xFF));
  }
  return true;
}

__device__ inline void split_four(uint64_t len, uint64_t* s, uint64_t* e) {
  uint64_t base = len / 4, rem = len % 4, start = 0;
  for (int i = 0; i < 4; ++i) {
    uint64_t l = base + ((uint64_t)i < rem ? 1 : 0);
    s[i] = start;
    e[i] = start + l;
    start += l;
  }
}

struct SharedHeader {
  uint64_t enc_off;   // offset of the entropy blob inside src
  uint64_t enc_len;
  uint32_t kind;      // 0 copy, 1 huffman, 2 rans, 3 empty-ok, 4 error
  uint32_t status;
  uint64_t copy_off;  // for kind 0
  uint32_t max_bits;
  uint32_t fixed;     // Huffman: every used symbol's code is max_bits long
  uint32_t nw;        // number of weights
  uint64_t seg_src[4];
  uint64_t seg_len[4];
  uint32_t err;
};

}  // namespace

// Parse the chunk frame and tag, decide what to run.  Executed by lane 0.
__device__ void parse_job(const DecodeJob& job, SharedHeader& h) {
  const uint8_t* src = reinterpret_cast<const uint8_t*>(job.src);
  uint64_t off = 0, len = job.src_len;
  h.status = kStOk;
  h.kind = 4;
  if (job.framed) {
    if (len < 5) { h.status = kStBadFrame; return; }
    uint64_t sl = ld_u32le(src + 1);
    if (len - 5 < sl) { h.status = kStBadFrame; return; }
    off = 5 + sl;
    len -= off;
  }
  if (job.codec == kCodecIdentity) {  // codecs/identity.rs: payload is the plane
    if (len != job.dst_len) { h.status = kStBadLength; return; }
    h.kind = 0;
    h.copy_off = off;
    return;
  }
  if (len == 0) { h.status = kStBadTag; return; }
  uint8_t tag = src[off];
  if (tag == 0) {                     // TAG_RAW
    if (len - 1 != job.dst_len) { h.status = kStBadLength; return; }
    h.kind = 0;
    h.copy_off = off + 1;
    return;
  }
  if (tag != 1) { h.status = kStBadTag; return; }
  if (len - 1 < 4) { h.status = kStBadTag; return; }
  uint64_t orig = ld_u32le(src + off + 1);
  uint64_t enc_len = len - 5;
  if (job.codec == kCodecHuffman) {
    if (orig > enc_len * 32 + 4096) { h.status = kStBadLength; return; }  // huffman.rs:122-131
    if (orig != job.dst_len) { h.status = kStBadLength; return; }
    h.kind = 1;
  } else if (job.codec == kCodecRans || job.codec == kCodecTans) {
    // rans.rs:158-160 / tans.rs:150-152 (check_within), then
    // length_prefix.rs:30-33 (tans.rs:118-126)
    if (orig > job.dst_len) { h.status = kStBadLength; return; }
    bool accepted = orig <= (1ull << 30) || orig <= enc_len * 64;
    if (!accepted) { h.status = kStBadLength; return; }
    if (orig == 0) {  // codec_tagged.rs:108-110; tans::decompress of 0 symbols
      h.kind = 3;
      if (job.dst_len != 0) h.status = kStBadLength;
      return;
    }
    if (orig != job.dst_len) { h.status = kStBadLength; return; }
    h.kind = job.codec == kCodecTans ? 5 : 2;
  } else {
    h.status = kStBadTag;
    return;
  }
  h.enc_off = off + 5;
  h.enc_len = enc_len;
}

// kRans: the rANS jobs (their own launch: its table entries and stream rings
// take three times the LDS of the other codecs), else every other job of
// this kernel.
template <bool kRans>
__global__ void __launch_bounds__(64) decode_exact_kernel(const DecodeJob* __restrict__ jobs,
                                                          uint32_t* __restrict__ status,
                                                          SyncStream* __restrict__ sync_streams,
                                                          uint16_t* __restrict__ sync_tables,
                                                          uint64_t* __restrict__ copy_src) {
  __shared__ SharedHeader h;
  __shared__ uint16_t rev[256];
  __shared__ uint8_t sorted_sym[256];              // Huffman: symbols by (length, symbol)
  // rANS: {freq | sym << 24, slot - start} per slot; tANS: one u32 per slot;
  // Huffman: (len << 8) | sym per window
  __shared__ __align__(16) uint32_t table_mem[(kRans ? 2 : 1) * kRansScale];
  __shared__ uint8_t hdr_stage[kHdrStage];   // Huffman: weights header and jump table
  uint2* table64 = reinterpret_cast<uint2*>(table_mem);
  uint32_t* table32 = table_mem;
  uint16_t* table16 = reinterpret_cast<uint16_t*>(table_mem);

  const uint32_t lane = threadIdx.x;
  const DecodeJob job = jobs[blockIdx.x];
  if (job.codec == kCodecZstd || job.codec == kCodecO1sac) return;  // zstd_decode_kernel's / o1sac_decode_kernel's job
  if ((job.codec == kCodecRans) != kRans) return;                    // the other instantiation's job
  const uint8_t* src = reinterpret_cast<const uint8_t*>(job.src);
  uint8_t* dst = reinterpret_cast<uint8_t*>(job.dst);

  if (lane == 0) {
    parse_job(job, h);
    h.err = 0;
  }
  __syncthreads();
  if (h.status != kStOk || h.kind == 3) {
    if (lane == 0) status[blockIdx.x] = h.status;
    return;
  }
  if (h.kind == 0) {  // stored bytes
    const uint8_t* s = src + h.copy_off;
    if (copy_src && job.dst_len >= kCopyDeferMin) {
      // large: copied by the parallel path's first pass or raw_copy_kernel, in pieces
      if (lane == 0) {
        copy_src[blockIdx.x] = reinterpret_cast<uint64_t>(s);
        status[blockIdx.x] = kStOk;
      }
      return;
    }
    for (uint64_t i = lane; i < job.dst_len; i += 64) g_st<uint8_t>((uint64_t)(dst + i), g_ld<uint8_t>((uint64_t)(s + i)));
    if (lane == 0) status[blockIdx.x] = kStOk;
    return;
  }
  const uint8_t* enc = src + h.enc_off;
  const uint64_t enc_len = h.enc_len;

  if constexpr (!kRans) {
  if (h.kind == 1) {
    // ---- weights header (weights.rs:34-85) and tree (tree.rs:87-177) ----
    // The header and jump table (at most 2 + 128 + 16 bytes) are staged in
    // LDS by the wavefront first.  Every lane then reads the header fields
    // (broadcast LDS reads) and the weights of symbols 4 lane .. 4 lane + 3;
    // lengths, counts and each symbol's rank among the symbols of its
    // length come from wave ballots, so the canonical code is built without
    // a serial pass over the 256 symbols.
    const uint8_t* const genc = enc;
    for (uint32_t i = lane; i < kHdrStage; i += 64) hdr_stage[i] = i < enc_len ? g_ld<uint8_t>((uint64_t)(genc + i)) : 0;
    __syncthreads();
    uint32_t st = kStOk;
    uint32_t n = 0, hb = 0;
    {
      const uint8_t b0 = hdr_stage[0];
      if (enc_len == 0 || !(b0 & 0x80)) st = kStBadHeader;
      else if (b0 == 0x80) {
        if (enc_len < 2) st = kStBadHeader;
        else {
          n = hdr_stage[1] ? hdr_stage[1] : 256;
          hb = 2;
          if (n < 128) st = kStBadHeader;
        }
      } else {
        n = b0 & 0x7F;
        hb = 1;
        if (n == 0) st = kStBadHeader;
      }
      if (st == kStOk && enc_len < hb + (n + 1) / 2) st = kStBadHeader;
    }
    uint32_t w[4] = {0, 0, 0, 0};
    if (st == kStOk) {
#pragma unroll
      for (uint32_t k = 0; k < 4; ++k) {
        const uint32_t i = 4 * lane + k;
        if (i < n) {
          const uint8_t b = hdr_stage[hb + i / 2];
          w[k] = (i % 2 == 0) ? (b & 0x0Fu) : ((b >> 4) & 0x0Fu);
        }
      }
    }
    const bool over = w[0] > (uint32_t)kHufMaxBits || w[1] > (uint32_t)kHufMaxBits ||
                      w[2] > (uint32_t)kHufMaxBits || w[3] > (uint32_t)kHufMaxBits;
    if (__ballot(over) != 0) st = kStBadHeader;
    // Per length: the symbol count (wave-uniform) and the rank of each of
    // the lane's symbols among the lower symbols of that length, from four
    // ballots.  Everything derived from the counts below is wave-uniform and
    // stays in scalar registers (constant indices in unrolled loops): no LDS
    // round trips and no serial lane-0 pass.
    uint32_t cnt[kHufMaxBits + 1];
    uint32_t rank[4] = {0, 0, 0, 0};
    cnt[0] = 0;
    {
      const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
      for (uint32_t l = 1; l <= (uint32_t)kHufMaxBits; ++l) {
        const uint64_t m0 = __ballot(w[0] == l), m1 = __ballot(w[1] == l), m2 = __ballot(w[2] == l),
                       m3 = __ballot(w[3] == l);
        const uint32_t r = __popcll(m0 & below) + __popcll(m1 & below) + __popcll(m2 & below) + __popcll(m3 & below);
        const uint32_t e0 = w[0] == l, e1 = w[1] == l, e2 = w[2] == l;
        if (w[0] == l) rank[0] = r;
        if (w[1] == l) rank[1] = r + e0;
        if (w[2] == l) rank[2] = r + e0 + e1;
        if (w[3] == l) rank[3] = r + e0 + e1 + e2;
        cnt[l] = __popcll(m0) + __popcll(m1) + __popcll(m2) + __popcll(m3);
      }
    }
    uint32_t maxb = 0;
#pragma unroll
    for (uint32_t l = 1; l <= (uint32_t)kHufMaxBits; ++l)
      if (cnt[l]) maxb = l;
    if (st == kStOk && maxb == 0) st = kStBadHeader;  // no symbol has a code
    if (maxb < 1) maxb = 1;
    // canonical codes (tree.rs:119-141): the first code of each length, with
    // the overflow checks the serial assignment makes; per length the index
    // of its first symbol in the symbols sorted by (length, symbol), and the
    // end of its left-aligned code range
    uint32_t sym_base[kHufMaxBits + 1], code_end[kHufMaxBits + 1];
    uint32_t shorter = 0;
    {
      uint32_t code = 0, base = 0;
      bool bad = false;
#pragma unroll
      for (uint32_t b = 1; b <= (uint32_t)kHufMaxBits; ++b) {
        sym_base[b] = 0;
        code_end[b] = 0;
        if (b <= maxb) {
          code = ((code + cnt[b - 1]) << 1) & 0xFFFF;
          bad |= code > (1u << b) || (cnt[b] && code + cnt[b] - 1 >= (1u << b));
          sym_base[b] = base;
          base += cnt[b];
          code_end[b] = (code + cnt[b]) << (maxb - b);
          if (b < maxb) shorter += cnt[b];
        }
      }
      if (st == kStOk && bad) st = kStBadHeader;
    }
    if (lane == 0) {
      h.fixed = st == kStOk && shorter == 0;
      // jump table and segment streams (decompress.rs:14-48)
      uint64_t pos = hb + (n + 1) / 2;
      if (st == kStOk && enc_len - pos < 16) st = kStBadHeader;
      if (st == kStOk) {
        uint64_t tot = 0, so = pos + 16;
        for (int i = 0; i < 4; ++i) {
          h.seg_len[i] = ld_u32le(hdr_stage + pos + 4 * i);
          h.seg_src[i] = so;
          so += h.seg_len[i];
          tot += h.seg_len[i];
        }
        if (tot != enc_len - pos - 16) st = kStBadHeader;
      }
      h.status = st;
      h.max_bits = maxb;
    }
    if (st == kStOk) {
#pragma unroll
      for (uint32_t k = 0; k < 4; ++k) {
        uint32_t sb = 0;
#pragma unroll
        for (uint32_t b = 1; b <= (uint32_t)kHufMaxBits; ++b)
          if (w[k] == b) sb = sym_base[b];
        if (w[k]) sorted_sym[sb + rank[k]] = (uint8_t)(4 * lane + k);
      }
    }
    __syncthreads();
    if (h.status != kStOk) {
      if (lane == 0) status[blockIdx.x] = h.status;
      return;
    }
    // table: index i holds the next max_bits stream bits, first bit lowest;
    // reversed, it is the left-aligned code value v.  The codes of length l
    // take v in [code_end[l - 1], code_end[l]), each symbol 2^(max_bits - l)
    // consecutive values in symbol order; the values past the last range
    // (an incomplete code) hold the fallback entry.  Filled length by
    // length, a value per lane.
    const uint32_t max_bits = maxb;
    const uint32_t tsize = 1u << max_bits;
    const uint16_t fallback = (uint16_t)(max_bits << 8);
    uint32_t vstart = 0;
#pragma unroll
    for (uint32_t l = 1; l <= (uint32_t)kHufMaxBits; ++l) {
      if (l <= max_bits) {
        const uint32_t vend = code_end[l], sh = max_bits - l, sb = sym_base[l];
        for (uint32_t v = vstart + lane; v < vend; v += 64)
          table16[__builtin_bitreverse32(v) >> (32 - max_bits)] =
              (uint16_t)((l << 8) | sorted_sym[sb + ((v - vstart) >> sh)]);
        vstart = vend;
      }
    }
    for (uint32_t v = vstart + lane; v < tsize; v += 64) table16[__builtin_bitreverse32(v) >> (32 - max_bits)] = fallback;
    __syncthreads();

    if (job.sync_id) {
      // parallel path: publish the table and the four streams, stop here
      const uint32_t d = job.sync_id - 1;
      for (uint32_t i = lane; i < tsize; i += 64) sync_tables[(uint64_t)kSyncTableEntries * d + i] = table16[i];
      if (lane < 4) {
        uint64_t s4[4], e4[4];
        split_four(job.dst_len, s4, e4);
        const uint32_t sb = job.pad[3];  // subsequence bits, chosen by the host
        uint32_t sub = job.sync_sub0;
        for (int i = 0; i < (int)lane; ++i) sub += (uint32_t)((h.seg_len[i] * 8 + sb - 1) / sb);
        SyncStream S;
        S.src = job.src + h.enc_off + h.seg_src[lane];
        S.m = h.seg_len[lane];
        S.dst = job.dst + s4[lane];
        S.n = e4[lane] - s4[lane];
        S.sub_bits = sb;
        S.reserved = 0;
        S.job = blockIdx.x;
        S.first_sub = sub;
        S.n_sub = (uint32_t)((h.seg_len[lane] * 8 + sb - 1) / sb);
        S.max_bits = (uint16_t)max_bits;
        S.fixed_len = h.fixed ? (uint16_t)max_bits : (uint16_t)0;
        S.table = d;
        S.pad = 0;
        sync_streams[4ull * d + lane] = S;
      }
      if (lane == 0) status[blockIdx.x] = kStDeferred;
      return;
    }

    if (lane < 4) {
      Reader r;
      rd_init(r, enc + h.seg_src[lane], h.seg_len[lane]);
      uint64_t s4[4], e4[4];
      split_four(job.dst_len, s4, e4);
      uint64_t op = s4[lane], end = e4[lane];
      uint64_t fe = end >= 3 ? end - 3 : 0;
      const uint64_t mask = (1ull << max_bits) - 1;
      // lockstep fast loop: continues only while all four streams qualify
      for (;;) {
        bool ok = op < fe && r.bi >= 3;
        uint64_t b = __ballot(ok);
        if ((b & 0xFull) != 0xFull) break;
#pragma unroll
        for (int round = 0; round < 2; ++round) {
          rd_refill(r);
          g_st<uint8_t>((uint64_t)(dst + op), rd_decode(r, table16, mask));
          g_st<uint8_t>((uint64_t)(dst + op + 1), rd_decode(r, table16, mask));
          op += 2;
        }
      }
      bool good = huf_tail(r, table16, mask, max_bits, dst + op, end - op);
      good = good && (r.bi < 0 && r.cont == 0);   // is_exhausted
      if (!good) atomicOr(&h.err, 1u);
    }
    __syncthreads();
    if (lane == 0) status[blockIdx.x] = h.err ? kStBadStream : kStOk;
    return;
  }

  if (h.kind == 5) return;  // tans_decode_kernel's job
  if (lane == 0) status[blockIdx.x] = kStBadTag;  // not reached: parse_job gives rANS jobs kind 2
  return;
  } else {
  // ---- rANS (rans/decompress.rs) ----
  if (lane == 0) {
    uint32_t st = kStOk;
    uint64_t max_sym = 0, need = 0;
    if (enc_len == 0) st = kStBadHeader;
    else {
      max_sym = enc[0];
      need = 1 + 2 * (max_sym + 1);
      if (enc_len < need) st = kStBadHeader;
    }
    uint32_t tot = 0;
    if (st == kStOk) {
      for (uint64_t i = 0; i < 256; ++i) {
        uint32_t f = i <= max_sym ? ((uint32_t)enc[1 + 2 * i] | ((uint32_t)enc[2 + 2 * i] << 8)) : 0;
        rev[i] = (uint16_t)f;   // reuse: per-symbol frequency
        tot += f;
      }
      if (tot != kRansScale) st = kStBadHeader;
    }
    if (st == kStOk && enc_len - need < 16) st = kStBadHeader;
    if (st == kStOk) {
      uint64_t t = 0, so = need + 16;
      for (int i = 0; i < 4; ++i) {
        h.seg_len[i] = ld_u32le(enc + need + 4 * i);
        h.seg_src[i] = so;
        so += h.seg_len[i];
        t += h.seg_len[i];
      }
      if (t != enc_len - need - 16) st = kStBadHeader;
    }
    h.status = st;
  }
  __syncthreads();
  if (h.status != kStOk) {
    if (lane == 0) status[blockIdx.x] = h.status;
    return;
  }
  // cumulative starts: lane 0 (256 adds), then parallel fill
  __shared__ uint16_t cum[257];
  if (lane == 0) {
    uint32_t run = 0;
    for (int s = 0; s < 256; ++s) { cum[s] = (uint16_t)run; run += rev[s]; }
    cum[256] = (uint16_t)run;
  }
  __syncthreads();
  // slot i of symbol s: {freq | s << 24, i - start}, so that one 24-bit
  // multiply-add, freq * (x >> 11) + (i - start), is the state update
  for (uint32_t s = lane; s < 256; s += 64) {
    const uint32_t f = rev[s], st = cum[s];
    for (uint32_t j = 0; j < f; ++j) table64[st + j] = make_uint2(f | (s << 24), j);
  }
  // Four lanes run the four serial state chains (decompress.rs:80-111).
  __shared__ __align__(16) uint8_t ring[4][kRansRing + kRansRingPad];
  uint64_t s4[4], e4[4];
  split_four(job.dst_len, s4, e4);
  const uint32_t c = lane & 3;
  const uint32_t sl = (uint32_t)h.seg_len[c];  // jump-table lengths are u32
  uint32_t k = (uint32_t)s4[c];
  const uint32_t end = (uint32_t)e4[c];
  const uint64_t out = reinterpret_cast<uint64_t>(dst);
  uint32_t x = 0, q = 4;  // state; next stream byte to read
  bool good = true, done = true, pending = false;
  if (lane < 4 && k != end) {
    if (sl < 4) good = false;
    else {
      const uint8_t* st = enc + h.seg_src[c];
      x = (uint32_t)g_ld<uint8_t>((uint64_t)st) | ((uint32_t)g_ld<uint8_t>((uint64_t)st + 1) << 8) |
          ((uint32_t)g_ld<uint8_t>((uint64_t)st + 2) << 16) | ((uint32_t)g_ld<uint8_t>((uint64_t)st + 3) << 24);
      done = false;
    }
  }
  // Staging, as every lane sees it: lane l loads granules (l & 15) and
  // (l & 15) + 16 of the next ones of chain l >> 4 (of four; lanes 0-63).
  // A granule is the 16-byte aligned global block g of the segment (its
  // byte o is at absolute index o + (address & 15)); aligned blocks that
  // hold a byte of the segment never cross a page, so reading the whole
  // block is in bounds.  A granule goes to ring slot (16 g) mod kRansRing
  // only once every byte that slot held has been consumed.
  const uint32_t sc = lane >> 4, su = lane & 15;
  const uint64_t sbase = reinterpret_cast<uint64_t>(enc + h.seg_src[sc]);
  const uint32_t soff = (uint32_t)(sbase & 15u);
  const uint64_t sgbase = sbase - soff;
  const uint32_t s_end_g = (uint32_t)((h.seg_len[sc] + soff + 15) / 16);
  uint32_t s_staged = 0;  // granules of chain sc staged so far (uniform per 16 lanes)
  uint8_t* const my_ring = ring[c];
  const uint32_t my_off = (uint32_t)((reinterpret_cast<uint64_t>(enc + h.seg_src[c])) & 15u);
  __syncthreads();  // table and ring addresses in place
  for (;;) {
    // this round's loads: chain sc's consumption point and done flag from lane sc
    const uint32_t q_c = (uint32_t)__shfl(q, (int)sc, 64);
    const bool done_c = __shfl((int)done, (int)sc, 64) != 0;
    const uint32_t lim = (q_c + soff) / 16 + kRansRing / 16 - 1;  // first granule whose slot is not free
    const uint32_t upto = done_c ? s_staged : min(min(lim, s_end_g), s_staged + kRansStageGranules);
    const uint32_t g0 = s_staged + su, g1 = g0 + 16;
    u32x4 v0 = u32x4_make(0, 0, 0, 0), v1 = v0;
    if (g0 < upto) v0 = g_ld<u32x4>(sgbase + 16ull * g0);
    if (g1 < upto) v1 = g_ld<u32x4>(sgbase + 16ull * g1);
    // decode what is staged: stream bytes [.., avail) of this lane's chain
    const uint32_t sg_mine = (uint32_t)__shfl((int)s_staged, (int)(16 * c), 64);
    const bool any = __ballot(lane < 4 && !done) != 0;
    if (lane < 4 && !done) {
      const uint32_t avail = sg_mine ? min(16 * sg_mine - my_off, sl) : 0u;
      uint32_t n = 0;
      auto rb = [&](uint32_t o) -> uint32_t { return my_ring[(o + my_off) & (kRansRing - 1)]; };
      for (;;) {
        if (pending) {  // careful renormalisation after a careful symbol (decompress.rs:104-107)
          bool suspend = false;
          while (x < kRansL) {
            if (q >= sl) { good = false; done = true; break; }
            if (q >= avail) { suspend = true; break; }
            x = (x << 8) | rb(q);
            ++q;
          }
          if (done || suspend) break;
          pending = false;
        }
        // Fast stretch: a normalised state (x >= L) decodes to at least
        // x >> 11 >= 2^12, so at most two bytes renormalise it; with two
        // staged bytes per step in hand the state stays normalised through
        // the stretch and needs no checks.  One byte is taken when the
        // decoded x1 < 2^23, a second when (x1 << 8 | b0) < 2^23, i.e.
        // x1 < 2^15.
        if (x >= kRansL) {
          uint32_t m = min(end - k, kRansRound - n);
          m = min(m, (avail - min(q, avail)) / 2);
          n += m;
          // Straight-line step: the bytes renormalising x1 are its leading
          // zero count rounded down to whole bytes (clz(x1) - 1 in 1..18 for
          // x1 in [2^12, 2^31)), shifted in from the top of the next two
          // stream bytes in one 64-bit shift.  qb is the ring read position
          // in bits.
          uint32_t qb = 8 * (q + my_off);
          auto step = [&]() -> uint32_t {
            const uint32_t idx = x & (kRansScale - 1);
            const uint2 e = table64[idx];
            uint16_t b01;
            __builtin_memcpy(&b01, my_ring + __builtin_amdgcn_ubfe(qb, 3, 11), 2);
            const uint32_t x1 = __umul24(e.x, x >> kRansProbBits) + e.y;
            const uint32_t sh = ((uint32_t)__builtin_clz(x1) - 1u) & ~7u;
            // [b0 b1 0 0] from the top byte down
            const uint32_t w = __builtin_amdgcn_perm(0u, (uint32_t)b01, 0x00010C0Cu);
            x = (uint32_t)(((((uint64_t)x1 << 32) | w) << sh) >> 32);
            qb += sh;
            return e.x;
          };
          // single steps up to a 4-byte aligned output address, then whole
          // output words of four symbols, then single steps
          for (; m && ((out + k) & 3u); --m, ++k) g_st<uint8_t>(out + k, (uint8_t)(step() >> 24));
          for (; m >= 4; m -= 4, k += 4) {
            // the symbols are the entries' top bytes: [a3 b3 d3 f3], low byte first
            const uint32_t a = step(), b = step(), d = step(), f = step();
            const uint32_t w = __builtin_amdgcn_perm(b, a, 0x0C0C0703u) | __builtin_amdgcn_perm(f, d, 0x07030C0Cu);
            g_st<uint32_t>(out + k, w);
          }
          for (; m; --m, ++k) g_st<uint8_t>(out + k, (uint8_t)(step() >> 24));
          q = qb / 8 - my_off;
        }
        // here pending is false: the last symbol's renormalisation is complete
        if (k == end) { done = true; break; }
        if (n >= kRansRound) break;
        // one careful symbol (unnormalised start, or the staged bytes' end)
        const uint32_t idx = x & (kRansScale - 1);
        const uint2 e = table64[idx];
        g_st<uint8_t>(out + k, (uint8_t)(e.x >> 24));
        x = __umul24(e.x, x >> kRansProbBits) + e.y;
        ++k;
        ++n;
        pending = true;
      }
    }
    if (!any) break;
    // this round's granules into the rings (after the decode: their slots
    // held bytes consumed before the round began)
    if (g0 < upto) {
      *reinterpret_cast<u32x4*>(&ring[sc][(16 * g0) & (kRansRing - 1)]) = v0;
      if (((16 * g0) & (kRansRing - 1)) == 0) *reinterpret_cast<u32x4*>(&ring[sc][kRansRing]) = v0;
    }
    if (g1 < upto) {
      *reinterpret_cast<u32x4*>(&ring[sc][(16 * g1) & (kRansRing - 1)]) = v1;
      if (((16 * g1) & (kRansRing - 1)) == 0) *reinterpret_cast<u32x4*>(&ring[sc][kRansRing]) = v1;
    }
    s_staged = max(s_staged, upto);
    __syncthreads();
  }
  if (lane < 4 && !good) atomicOr(&h.err, 1u);
  __syncthreads();
  if (lane == 0) status[blockIdx.x] = h.err ? kStBadStream : kStOk;
  }
}

// tANS payloads: one serial state chain each.  The job is parsed as
// decode_exact_kernel parses it; that kernel reports every other outcome of
// a tANS job (refusals, stored payloads, empty planes), this one the chains.
__global__ void __launch_bounds__(64) tans_decode_kernel(const DecodeJob* __restrict__ jobs,
                                                         uint32_t* __restrict__ status) {
  __shared__ SharedHeader h;
  __shared__ uint16_t rev[256];
  __shared__ uint8_t sorted_sym[256];
  __shared__ __align__(16) uint32_t table32[2048];
  const uint32_t lane = threadIdx.x;
  const DecodeJob job = jobs[blockIdx.x];
  if (job.codec != kCodecTans) return;
  if (lane == 0) parse_job(job, h);
  __syncthreads();
  if (h.status != kStOk || h.kind != 5) return;
  uint8_t* dst = reinterpret_cast<uint8_t*>(job.dst);
  const uint8_t* enc = reinterpret_cast<const uint8_t*>(job.src) + h.enc_off;
  const uint64_t enc_len = h.enc_len;
  // ---- tANS (entropy/tans/mod.rs:372-455): one serial state chain ----
  // Header: table_log 11, nsym in 2..=256, (sym u8, freq u16) pairs with no
  // repeat and no zero summing to L = 2048, total_bits u64 <= 8 x stream.
  // The wavefront parses it (four entries per lane; a repeat shows as a
  // symbol whose owner slot names another entry), builds the decode table
  // slot-parallel, then runs the state chain with wave-uniform state.
  __shared__ uint16_t tcum[256];
  __shared__ __align__(16) uint32_t tstage[kTansStageWords];
  uint8_t* const owner = sorted_sym;  // reuse: the entry that names a symbol
  for (uint32_t s = lane; s < 256; s += 64) rev[s] = 0;  // reuse: normalized frequency per symbol
  uint32_t nsym = 0;
  bool hok = enc_len >= 3 && g_ld<uint8_t>((uint64_t)enc) == 11;
  if (hok) {
    nsym = g_ld<uint8_t>((uint64_t)(enc + 1)) | ((uint32_t)g_ld<uint8_t>((uint64_t)(enc + 2)) << 8);
    hok = nsym >= 2 && nsym <= 256 && 3 + 3 * (uint64_t)nsym + 8 <= enc_len;
  }
  uint32_t es[4], ef[4];
#pragma unroll
  for (uint32_t k = 0; k < 4; ++k) {
    const uint32_t i = lane + 64 * k;
    es[k] = 0;
    ef[k] = 0;
    if (hok && i < nsym) {
      const uint8_t* e = enc + 3 + 3 * i;
      es[k] = g_ld<uint8_t>((uint64_t)e);
      ef[k] = g_ld<uint8_t>((uint64_t)(e + 1)) | ((uint32_t)g_ld<uint8_t>((uint64_t)(e + 2)) << 8);
    }
  }
  __syncthreads();
#pragma unroll
  for (uint32_t k = 0; k < 4; ++k)
    if (hok && lane + 64 * k < nsym) owner[es[k]] = (uint8_t)(lane + 64 * k);
  __syncthreads();
  bool bad = false;
  uint32_t sum = 0;
#pragma unroll
  for (uint32_t k = 0; k < 4; ++k) {
    if (hok && lane + 64 * k < nsym) {
      bad |= owner[es[k]] != (uint8_t)(lane + 64 * k) || ef[k] == 0;  // a repeat, or a zero
      sum += ef[k];
      rev[es[k]] = (uint16_t)ef[k];
    }
  }
  uint64_t tb = 0;
  const uint64_t bs_off = 3 + 3 * (uint64_t)nsym + 8;
  if (hok) {
#pragma unroll
    for (int k = 7; k >= 0; --k) tb = (tb << 8) | g_ld<uint8_t>((uint64_t)(enc + bs_off - 8 + (uint64_t)k));
  }
  hok = hok && __ballot(bad) == 0 && wave_sum_u32(sum) == 2048 && tb <= (enc_len - bs_off) * 8;
  if (!hok) {
    if (lane == 0) status[blockIdx.x] = kStBadHeader;
    return;
  }
  __syncthreads();
  {
    uint32_t c[4], t = 0;
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) t += (c[k] = rev[4 * lane + k]);
    uint32_t run = wave_excl_sum_u32(t);
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) {
      tcum[4 * lane + k] = (uint16_t)run;
      run += c[k];
    }
  }
  __syncthreads();
  // spread (mod.rs:199-211): the k-th placement, in symbol order, lands on
  // slot k (L/2 + L/8 + 3) mod L; the step is odd, so every slot once
  for (uint32_t s = lane; s < 256; s += 64)
    for (uint32_t k = tcum[s], e = tcum[s] + rev[s]; k < e; ++k) table32[(k * 1283u) & 2047u] = s;
  __syncthreads();
  // build_decode (mod.rs:346-368): slots in order; the occurrence x of the
  // slot's symbol runs from norm[s] to 2 norm[s] - 1.  64 slots a round:
  // a slot's x is its symbol's count so far plus the lanes below it with
  // the same symbol (eight ballots find them); the group's last lane
  // advances the count.
  for (uint32_t u0 = 0; u0 < 2048; u0 += 64) {
    const uint32_t u = u0 + lane;
    const uint32_t sy = table32[u] & 255u;
    uint64_t same = ~0ull;
#pragma unroll
    for (uint32_t bit = 0; bit < 8; ++bit) {
      const uint64_t bl = __ballot((sy >> bit) & 1u);
      same &= ((sy >> bit) & 1u) ? bl : ~bl;
    }
    const uint64_t below = same & ((1ull << lane) - 1ull);
    const uint32_t x = rev[sy] + (uint32_t)__popcll(below);
    __builtin_amdgcn_wave_barrier();
    if ((same >> lane) == 1ull) rev[sy] = (uint16_t)(x + 1);
    const uint32_t nb = 11u - (31u - (uint32_t)__builtin_clz(x));
    table32[u] = sy | (nb << 8) | (((x << nb) - 2048u) << 16);
    __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();
  // LIFO reader (mod.rs:102-150): pops the nb bits below `pos` (bit i of
  // the stream is bit i & 7 of byte i >> 3).  The stream is staged in LDS
  // as 32-bit words, kTansStageWords at a time from its end down; a 64-bit
  // register window holds bits [32 wi, 32 wi + 64) and takes the next
  // lower word (read one refill earlier) when fewer than 32 bits lie below
  // pos.  The decode table sits in registers: entry u in register u / 64
  // of lane u % 64, read by a register-indexed move and a lane read.
  const uint8_t* bs = enc + bs_off;
  const uint64_t bl = enc_len - bs_off;
  const int64_t top = tb ? (int64_t)((tb - 1) >> 5) : -1;  // word holding bit tb - 1
  int64_t stage_lo = top >= 0 ? top / kTansStageWords * kTansStageWords : 0;  // first word staged
  auto stage = [&]() {  // words stage_lo.. ; bytes past the stream read as zero
    __syncthreads();
    if (bl == 0) {
      for (uint32_t j = lane; j < kTansStageWords; j += 64) tstage[j] = 0;
    } else {
#pragma unroll 4
      for (uint32_t j = lane; j < kTansStageWords; j += 64) {
        const uint64_t b0 = 4ull * ((uint64_t)stage_lo + j);
        uint32_t v = 0;
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q) {
          const uint32_t x = g_ld<uint8_t>((uint64_t)(bs + (b0 + q < bl ? b0 + q : bl - 1)));
          v |= (b0 + q < bl ? x : 0u) << (8 * q);
        }
        tstage[j] = v;
      }
    }
    __syncthreads();
  };
  // word w of the stream as read from the stage (0 below the stream); the
  // value is a vector register, made wave-uniform where it is used
  auto word = [&](int64_t w) -> uint32_t {
    if (w < 0) return 0u;
    if (w < stage_lo) {
      stage_lo -= kTansStageWords;
      stage();
    }
    return tstage[w - stage_lo];
  };
  stage();
  uint32_t tab[32];
#pragma unroll
  for (uint32_t r = 0; r < 32; ++r) tab[r] = table32[64 * r + lane];
  // the window starts at bit 32 wi (wi < 0: bits below the stream, zero);
  // rel = pos - 32 wi.  pos only decreases, so a pop below the stream's
  // start (pos < nb) leaves pos negative at the end: the chain runs on
  // through zero bits and the final check refuses it.
  int64_t wi = top - 1;
  const uint32_t w_top = __builtin_amdgcn_readfirstlane(word(top));
  uint64_t win = ((uint64_t)w_top << 32) | (uint32_t)__builtin_amdgcn_readfirstlane(word(top - 1));
  uint32_t next = word(top - 2);
  uint32_t rel = (uint32_t)(tb - 32 * (uint64_t)(top - 1));  // tb - 32 wi, in [33, 64] (tb > 0)
  // stage index of word wi - 1 (negative below the stage), so that a
  // refill compares 32-bit indices and restages only when it leaves the piece
  int32_t si = (int32_t)(wi - 1 - stage_lo);
  auto refill = [&]() {
    win = (win << 32) | (uint32_t)__builtin_amdgcn_readfirstlane(next);
    rel += 32;
    --wi;
    --si;
    if (si >= 0) {
      next = tstage[si];
    } else if (stage_lo > 0) {  // word wi - 1 = stage_lo - 1: the piece below
      stage_lo -= kTansStageWords;
      stage();
      si += (int32_t)kTansStageWords;
      next = tstage[si];
    } else {
      next = 0u;  // below the stream
    }
  };
  uint32_t state = 0;
  if (tb >= 11) {
    rel -= 11;
    state = (uint32_t)(win >> rel) & 2047u;
    if (rel < 32) refill();
  }
  // one step: the symbol of `state`, then its nb bits
  auto step = [&]() -> uint32_t {
    const uint32_t e = __builtin_amdgcn_readlane(tab[__builtin_amdgcn_readfirstlane(state >> 6)], state & 63u);
    const uint32_t nb = (e >> 8) & 15u;
    rel -= nb;  // rel >= 32 before the pop, nb <= 11
    state = (e >> 16) + ((uint32_t)(win >> rel) & ((1u << nb) - 1u));
    if (rel < 32) refill();
    return e & 255u;
  };
  uint8_t* const out = dst;
  const uint64_t n = tb >= 11 ? job.dst_len : 0;
  for (uint64_t i = 0; i < n; i += 256) {
    // 256 symbols a round, four to a lane's word
    const uint32_t m = n - i < 256 ? (uint32_t)(n - i) : 256u;
    uint32_t outv = 0, j = 0;
    for (; j + 4 <= m; j += 4) {
      uint32_t pk = step();
      pk |= step() << 8;
      pk |= step() << 16;
      pk |= step() << 24;
      outv = lane == (j >> 2) ? pk : outv;
    }
    if (j < m) {
      uint32_t pk = 0;
      for (uint32_t t = 0; j + t < m; ++t) pk |= step() << (8 * t);
      outv = lane == (j >> 2) ? pk : outv;
    }
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q)
      if (4 * lane + q < m) g_st<uint8_t>((uint64_t)(out + i + 4 * lane + q), (uint8_t)(outv >> (8 * q)));
  }
  const int64_t pos = tb >= 11 ? 32 * wi + (int64_t)rel : -1;
  bool good = true;
  // fully consumed and back at the start state (mod.rs:444-453)
  if (good && (pos != 0 || state != 0)) good = false;
  if (lane == 0) status[blockIdx.x] = good ? kStOk : kStBadStream;
  return;
}

hipError_t launch_decode_exact(const DecodeJob* jobs_dev, uint32_t* status_dev, uint32_t n_jobs,
                               SyncStream* sync_streams, uint16_t* sync_tables, uint64_t* copy_src,
                               hipStream_t stream) {
  if (n_jobs == 0) return hipSuccess;
  hipLaunchKernelGGL(decode_exact_kernel<false>, dim3(n_jobs), dim3(64), 0, stream, jobs_dev, status_dev, sync_streams,
                     sync_tables, copy_src);
  return hipGetLastError();
}

hipError_t launch_tans_decode(const DecodeJob* jobs_dev, uint32_t* status_dev, uint32_t n_jobs, hipStream_t stream) {
  if (n_jobs == 0) return hipSuccess;
  hipLaunchKernelGGL(tans_decode_kernel, dim3(n_jobs), dim3(64), 0, stream, jobs_dev, status_dev);
  return hipGetLastError();
}

hipError_t launch_rans_exact(const DecodeJob* jobs_dev, uint32_t* status_dev, uint32_t n_jobs, uint64_t* copy_src,
                             hipStream_t stream) {
  if (n_jobs == 0) return hipSuccess;
  hipLaunchKernelGGL(decode_exact_kernel<true>, dim3(n_jobs), dim3(64), 0, stream, jobs_dev, status_dev, nullptr,
                     nullptr, copy_src);
  return hipGetLastError();
}

}  // namespace ptwm
