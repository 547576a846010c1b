// huff_ilv.hip -- the GPU-native interleaved Huffman plane codec on gfx950.
//
// Wire format (codec wire id 0x7F01, this library's plane-codec id):
//   [tag u8] 0: stored plane bytes follow.  1: coded:
//   [orig_len u32 LE][weights header (entropy/huffman/weights.rs)][0-pad to 4]
//   [block offset table u32 x (nb + 1)][data],  nb = ceil(n / 16384)
//   block b = data[off[b] .. off[b+1]):
//     [64 x u8 lane word counts][lane 0 words][lane 1 words]...  (u32 LE)
//   lane j codes the 16-symbol groups g = j + 64 r (r = 0..15) of its block,
//   group g = plane positions [16384 b + 16 g, +16) (clipped to n), as the
//   reference's bit-reversed canonical codes (tree.rs:102-177) packed
//   LSB-first.  Acceptance: each lane's word count == ceil(bits used / 32).
//
// Decode: one wavefront per block.  In round r every lane decodes one group,
// so a round's 64 groups are 1024 consecutive symbols and the merged output
// of a round is one contiguous span: all stores are coalesced dwordx4.  An
// 11-bit multi-symbol lookup table in LDS (up to 3 symbols per lookup) is
// built per workgroup from the payload's weights header.  Tensors whose
// planes are all stored-aligned or huff_ilv-coded are decoded and merged in
// one pass (decode -> inverse chain -> store), so planes never round-trip
// through HBM.
//
// Encode: LDS-privatised histograms merged with atomics, host code-table
// build (256 symbols), a size pass (one wave per block: per-lane bit counts
// from the code lengths), a host prefix sum for block offsets, and an encode
// pass that writes each lane's words at its prefix-summed offset.
#include "huff_ilv.h"

#include <cstring>

namespace ptwm {

namespace {

__device__ __forceinline__ uint32_t revert16x2(uint32_t v) {
  return ((v << 8) & 0x80008000u) | ((v >> 1) & 0x7F807F80u) | (v & 0x007F007Fu);
}
__device__ __forceinline__ uint32_t revert32(uint32_t v) {
  return ((v << 8) & 0x80000000u) | ((v >> 1) & 0x7F800000u) | (v & 0x007FFFFFu);
}
__device__ __forceinline__ uint32_t revert_e4m3x4(uint32_t r) {
  return ((r & 0xF0F0F0F0u) >> 1) | ((r & 0x08080808u) << 4) | (r & 0x07070707u);
}
__device__ __forceinline__ uint32_t revert_e5m2x4(uint32_t r) {
  return ((r & 0xF8F8F8F8u) >> 1) | ((r & 0x04040404u) << 5) | (r & 0x03030303u);
}
__device__ __forceinline__ void zip2(uint32_t a, uint32_t b, uint32_t& lo, uint32_t& hi) {
  lo = __builtin_amdgcn_perm(b, a, 0x05010400u);
  hi = __builtin_amdgcn_perm(b, a, 0x07030602u);
}
__device__ __forceinline__ uint32_t ld_u32le(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// inclusive prefix sum across the 64 lanes of a wavefront
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  const uint32_t lane = threadIdx.x & 63u;
#pragma unroll
  for (uint32_t d = 1; d < 64; d <<= 1) {
    uint32_t t = __shfl_up(v, d, 64);
    if (lane >= d) v += t;
  }
  return v;
}

// Per-coded-plane decode tables, resident in LDS for the whole workgroup.
struct LutSet {
  uint32_t lut[2048];   // s0 | s1 << 8 | s2 << 16 | n << 24 | bits << 26 | fb0 << 30 | fb1 << 31
  uint8_t len[256];     // code length per symbol
  uint32_t max_bits;
  uint32_t status;
  uint32_t pad[2];
};
// Build-time scratch, shared by every plane of the workgroup.
struct BuildScratch {
  uint16_t t16[2048];   // single-symbol table (len << 8 | sym), tree.rs:143-169
  uint16_t rev[256];
  uint32_t counts[16];
  uint32_t next_code[16];
  uint32_t wave_len_count[4][16];
  uint32_t nw, hb, err, hdr_len;
};

// Build the tables of one plane from the weights header at hdr (hdr_avail
// bytes readable).  All 256 threads of the workgroup take part.  Sets
// ls.status (nonzero: invalid header) and bs.hdr_len.
__device__ void build_tables(LutSet& ls, BuildScratch& bs, const uint8_t* hdr, uint64_t hdr_avail) {
  const uint32_t t = threadIdx.x;
  if (t == 0) {
    uint32_t err = 0, n = 0, hb = 0;
    if (hdr_avail < 1 || !(hdr[0] & 0x80)) err = 1;
    else if (hdr[0] == 0x80) {
      if (hdr_avail < 2) err = 1;
      else {
        n = hdr[1] ? hdr[1] : 256;
        hb = 2;
        if (n < 128) err = 1;
      }
    } else {
      n = hdr[0] & 0x7F;
      hb = 1;
      if (n == 0) err = 1;
    }
    if (!err && hdr_avail < hb + (n + 1) / 2) err = 1;
    bs.nw = n;
    bs.hb = hb;
    bs.err = err;
    bs.hdr_len = hb + (n + 1) / 2;
  }
  __syncthreads();
  const uint32_t n = bs.nw, hb = bs.hb;
  uint32_t w = 0;
  if (!bs.err && t < n) {
    uint8_t b = hdr[hb + t / 2];
    w = (t % 2 == 0) ? (b & 0x0F) : ((b >> 4) & 0x0F);
  }
  if (w > 11) atomicOr(&bs.err, 1u);
  if (w > 11) w = 0;
  ls.len[t] = (uint8_t)w;
  // rank among same-length symbols with a smaller index: ballots per length
  const uint32_t wave = t >> 6, lane = t & 63u;
  uint32_t rank_in_wave = 0;
  for (uint32_t l = 1; l <= 11; ++l) {
    uint64_t m = __ballot(w == l);
    if (w == l) rank_in_wave = __popcll(m & ((1ull << lane) - 1ull));
    if (lane == 0) bs.wave_len_count[wave][l] = __popcll(m);
  }
  __syncthreads();
  if (t == 0) {
    uint32_t maxb = 0, total = 0;
    bs.counts[0] = 0;
    for (uint32_t l = 1; l <= 11; ++l) {
      uint32_t c = 0;
      for (int wv = 0; wv < 4; ++wv) c += bs.wave_len_count[wv][l];
      bs.counts[l] = c;
      total += c;
      if (c) maxb = l;
    }
    if (total == 0) bs.err = 1;
    if (maxb < 1) maxb = 1;
    uint32_t code = 0;
    for (uint32_t b = 1; b <= maxb; ++b) {
      code = (code + bs.counts[b - 1]) << 1;
      if (code > (1u << b)) bs.err = 1;
      bs.next_code[b] = code;
    }
    // Kraft <= 1 (equivalent to the per-symbol c < 2^len checks of tree.rs)
    uint32_t kraft = 0;
    for (uint32_t l = 1; l <= maxb; ++l) kraft += bs.counts[l] << (11 - l);
    if (kraft > 2048) bs.err = 1;
    ls.max_bits = maxb;
  }
  __syncthreads();
  const uint32_t max_bits = ls.max_bits;
  if (w) {
    uint32_t before = 0;
    for (uint32_t wv = 0; wv < wave; ++wv) before += bs.wave_len_count[wv][w];
    uint32_t c = bs.next_code[w] + before + rank_in_wave;
    uint32_t r = 0;
    for (uint32_t k = 0; k < w; ++k) r |= ((c >> k) & 1u) << (w - 1 - k);
    bs.rev[t] = (uint16_t)r;
  } else {
    bs.rev[t] = 0;
  }
  const uint16_t fallback = (uint16_t)(max_bits << 8);
  for (uint32_t i = t; i < 2048; i += 256) bs.t16[i] = fallback;
  __syncthreads();
  if (!bs.err && w) {
    uint16_t e = (uint16_t)((w << 8) | t);
    uint32_t spread = 1u << (max_bits - w);
    for (uint32_t i = 0; i < spread; ++i) bs.t16[bs.rev[t] | (i << w)] = e;
  }
  __syncthreads();
  // multi-symbol entries: greedy decode of up to 3 whole codes in 11 bits
  const uint32_t mask = (1u << max_bits) - 1u;
  for (uint32_t i = t; i < 2048; i += 256) {
    uint32_t e0 = bs.t16[i & mask];
    uint32_t used = e0 >> 8, n_sym = 1, syms = e0 & 0xFF;
    uint32_t fb = (e0 == fallback && ls.len[0] != max_bits) ? (1u << 30) : 0u;
    uint32_t e1 = bs.t16[(i >> used) & mask];
    if ((e1 >> 8) <= 11 - used) {
      syms |= (e1 & 0xFF) << 8;
      fb |= (e1 == fallback && ls.len[0] != max_bits) ? (1u << 31) : 0u;
      used += e1 >> 8;
      n_sym = 2;
      uint32_t e2 = bs.t16[(i >> used) & mask];
      if ((e2 >> 8) <= 11 - used) {
        syms |= (e2 & 0xFF) << 16;
        used += e2 >> 8;
        n_sym = 3;
      }
    }
    ls.lut[i] = syms | (n_sym << 24) | (used << 26) | fb;
  }
  if (t == 0) ls.status = bs.err;
  __syncthreads();
}

// Plain global-memory load (the address arrives through LDS, so the
// compiler cannot infer the address space and would emit a flat load).
__device__ __forceinline__ uint32_t gload_u32(const uint32_t* p) {
  return *(const __attribute__((address_space(1))) uint32_t*)(uintptr_t)p;
}

// Decoder state of one coded plane within a block, per lane.  `nxt` holds
// the next stream word, loaded one refill ahead: the load is issued straight
// into `nxt` (no select on the value, which would force a wait), from the
// lane's stream or, past its end, from `safe` (the block's first word, always
// readable).  Words past the end are never part of an accepted stream: a lane
// whose symbols reach past its words consumes more than 32 * count bits and
// fails the word-count check, exactly as the specification decoder (which
// reads zeros there) does.
struct LaneBits {
  const uint32_t* ptr;
  const uint32_t* end;
  const uint32_t* safe;
  const uint32_t* start;
  uint64_t buf;
  uint32_t cnt;
  uint32_t nxt;
};

__device__ __forceinline__ void lane_start(LaneBits& lb, const uint32_t* ptr, const uint32_t* end,
                                           const uint32_t* safe) {
  lb.ptr = ptr;
  lb.start = ptr;
  lb.end = end;
  lb.safe = safe;
  lb.buf = 0;
  lb.cnt = 0;
  lb.nxt = gload_u32(lb.ptr < lb.end ? lb.ptr : lb.safe);
  lb.ptr++;
}

// bits consumed so far: words pulled into the buffer minus what it still holds
__device__ __forceinline__ uint32_t lane_used(const LaneBits& lb) {
  return 32u * (uint32_t)(lb.ptr - lb.start - 1) - lb.cnt;
}

// Decode `count` (<= 16) symbols of one group.  Symbols go to the lane's
// 20-byte LDS staging slot (three byte stores per lookup; bytes past the
// group land in the slot's padding) and come back as 4 words.
__device__ __forceinline__ void decode_group(const LutSet& ls, LaneBits& lb, uint32_t count, uint8_t* stage,
                                             uint32_t& w0, uint32_t& w1, uint32_t& w2, uint32_t& w3) {
  uint32_t produced = 0;
  while (produced < count) {
    if (lb.cnt < 32) {
      lb.buf |= (uint64_t)lb.nxt << lb.cnt;
      lb.cnt += 32;
      lb.nxt = gload_u32(lb.ptr < lb.end ? lb.ptr : lb.safe);
      lb.ptr++;
    }
    const uint32_t e = ls.lut[(uint32_t)lb.buf & 2047u];
    uint32_t n = (e >> 24) & 3u, bits = (e >> 26) & 15u;
    const uint32_t rem = count - produced;
    if (n > rem) {
      // group end inside this entry: lengths of the first one or two codes
      n = rem;
      bits = (e & (1u << 30)) ? ls.max_bits : ls.len[e & 0xFF];
      if (n == 2) bits += (e & (1u << 31)) ? ls.max_bits : ls.len[(e >> 8) & 0xFF];
    }
    lb.buf >>= bits;
    lb.cnt -= bits;
    stage[produced] = (uint8_t)e;
    stage[produced + 1] = (uint8_t)(e >> 8);
    stage[produced + 2] = (uint8_t)(e >> 16);
    produced += n;
  }
  const uint32_t* sw = reinterpret_cast<const uint32_t*>(stage);
  w0 = sw[0];
  w1 = sw[1];
  w2 = sw[2];
  w3 = sw[3];
}

// Lane state when the block's words are staged in LDS: word indexes into the
// wavefront's staging array instead of global pointers.
struct LaneLds {
  uint32_t off;
  uint32_t end;
  uint32_t start;
  uint32_t cnt;
  uint64_t buf;
  uint32_t nxt;
};

__device__ __forceinline__ void lane_start_lds(LaneLds& lb, const uint32_t* sw, uint32_t off, uint32_t end) {
  lb.off = off;
  lb.start = off;
  lb.end = end;
  lb.buf = 0;
  lb.cnt = 0;
  lb.nxt = sw[off < end ? off : 0u];
  lb.off++;
}

__device__ __forceinline__ uint32_t lane_used_lds(const LaneLds& lb) {
  return 32u * (lb.off - lb.start - 1u) - lb.cnt;
}

// decode_group with the lane's words read from LDS (sw: the wavefront's
// staged words; reads past the lane's end use word 0, see LaneBits).
__device__ __forceinline__ void decode_group_lds(const LutSet& ls, const uint32_t* sw, LaneLds& lb, uint32_t count,
                                                 uint8_t* stage, uint32_t& w0, uint32_t& w1, uint32_t& w2,
                                                 uint32_t& w3) {
  uint32_t produced = 0;
  while (produced < count) {
    if (lb.cnt < 32) {
      lb.buf |= (uint64_t)lb.nxt << lb.cnt;
      lb.cnt += 32;
      lb.nxt = sw[lb.off < lb.end ? lb.off : 0u];
      lb.off++;
    }
    const uint32_t e = ls.lut[(uint32_t)lb.buf & 2047u];
    uint32_t n = (e >> 24) & 3u, bits = (e >> 26) & 15u;
    const uint32_t rem = count - produced;
    if (n > rem) {
      n = rem;
      bits = (e & (1u << 30)) ? ls.max_bits : ls.len[e & 0xFF];
      if (n == 2) bits += (e & (1u << 31)) ? ls.max_bits : ls.len[(e >> 8) & 0xFF];
    }
    lb.buf >>= bits;
    lb.cnt -= bits;
    stage[produced] = (uint8_t)e;
    stage[produced + 1] = (uint8_t)(e >> 8);
    stage[produced + 2] = (uint8_t)(e >> 16);
    produced += n;
  }
  const uint32_t* st = reinterpret_cast<const uint32_t*>(stage);
  w0 = st[0];
  w1 = st[1];
  w2 = st[2];
  w3 = st[3];
}

static_assert(sizeof(BuildScratch) <= kIlvScratchBytes, "scratch layout");

}  // namespace

// ---------------------------------------------------------------------------
// decode (fused with the inverse chain)
// ---------------------------------------------------------------------------

template <uint32_t kChain>
struct ChainInfo;
template <> struct ChainInfo<kChainIeee16Split2> { static constexpr uint32_t np = 2, ratio = 2; };
template <> struct ChainInfo<kChainIeee32Split4> { static constexpr uint32_t np = 4, ratio = 4; };
template <> struct ChainInfo<kChainE4m3Nibble> { static constexpr uint32_t np = 2, ratio = 1; };
template <> struct ChainInfo<kChainE5m2Nibble> { static constexpr uint32_t np = 2, ratio = 1; };
template <> struct ChainInfo<kChainNibbleSplit> { static constexpr uint32_t np = 2, ratio = 1; };
template <> struct ChainInfo<kChainPassthrough> { static constexpr uint32_t np = 1, ratio = 1; };

// Merge one group (16 elements; v[p][k] = plane p bytes 4k..4k+3) into the
// output words o[] (ratio * 4 words).
template <uint32_t kChain>
__device__ __forceinline__ void merge_group(const uint32_t (&v)[ChainInfo<kChain>::np][4],
                                            uint32_t (&o)[4 * ChainInfo<kChain>::ratio]) {
  if constexpr (kChain == kChainIeee16Split2) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t lo, hi;
      zip2(v[0][k], v[1][k], lo, hi);
      o[2 * k] = revert16x2(lo);
      o[2 * k + 1] = revert16x2(hi);
    }
  } else if constexpr (kChain == kChainIeee32Split4) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t ab_lo, ab_hi, cd_lo, cd_hi;
      zip2(v[0][k], v[1][k], ab_lo, ab_hi);
      zip2(v[2][k], v[3][k], cd_lo, cd_hi);
      o[4 * k + 0] = revert32(__builtin_amdgcn_perm(cd_lo, ab_lo, 0x05040100u));
      o[4 * k + 1] = revert32(__builtin_amdgcn_perm(cd_lo, ab_lo, 0x07060302u));
      o[4 * k + 2] = revert32(__builtin_amdgcn_perm(cd_hi, ab_hi, 0x05040100u));
      o[4 * k + 3] = revert32(__builtin_amdgcn_perm(cd_hi, ab_hi, 0x07060302u));
    }
  } else if constexpr (kChain == kChainPassthrough) {
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = v[0][k];
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t r8 = ((v[0][k] & 0x0F0F0F0Fu) << 4) | (v[1][k] & 0x0F0F0F0Fu);
      if constexpr (kChain == kChainE4m3Nibble) o[k] = revert_e4m3x4(r8);
      else if constexpr (kChain == kChainE5m2Nibble) o[k] = revert_e5m2x4(r8);
      else o[k] = r8;
    }
  }
}

template <uint32_t kChain>
__global__ void __launch_bounds__(256) ilv_decode_kernel(const IlvTensor* __restrict__ tensors,
                                                         const IlvTile* __restrict__ tiles,
                                                         uint32_t* __restrict__ status, uint32_t n_slots,
                                                         uint32_t stage_words) {
  constexpr uint32_t NP = ChainInfo<kChain>::np;
  constexpr uint32_t RATIO = ChainInfo<kChain>::ratio;
  // dynamic LDS: [LutSet x n_slots][byte staging: 256 lanes x 20 B]
  //              [word staging: 4 wavefronts x stage_words], the table-build
  //              scratch aliasing the word staging (built before any staging)
  extern __shared__ __align__(16) uint8_t smem[];
  LutSet* slots = reinterpret_cast<LutSet*>(smem);
  uint8_t* stage_base = smem + n_slots * sizeof(LutSet);
  uint32_t* word_stage = reinterpret_cast<uint32_t*>(stage_base + 256 * 20);
  BuildScratch& bs = *reinterpret_cast<BuildScratch*>(word_stage);
  __shared__ uint64_t s_table[NP], s_data[NP], s_datalen[NP], s_raw[NP];
  __shared__ uint32_t s_bad, s_slot[NP];   // s_slot: 0 = not coded, k = slot k - 1
  const IlvTile tile = tiles[blockIdx.x];
  const IlvTensor& T = tensors[tile.tensor];
  const uint32_t t = threadIdx.x;
  const uint64_t n = T.n;
  const uint32_t nb = (uint32_t)((n + kIlvBlock - 1) / kIlvBlock);
  if (t == 0) {
    s_bad = 0;
    uint32_t next_slot = 0;
    for (uint32_t p = 0; p < NP; ++p) {
      const IlvPlane& P = T.planes[p];
      s_raw[p] = P.base;
      s_slot[p] = 0;
      if (!P.coded) continue;
      // huff_ilv payload: tag 0 stores the plane after the tag byte
      const uint8_t* pay = reinterpret_cast<const uint8_t*>(P.base);
      if (P.len == 0) s_bad |= kIlvErrHeader;
      else if (pay[0] == 0) {
        if (P.len != n + 1) s_bad |= kIlvErrHeader;
        s_raw[p] = P.base + 1;
      } else if (pay[0] == 1 && P.len >= 5 && ld_u32le(pay + 1) == n) {
        if (next_slot < n_slots) s_slot[p] = ++next_slot;
        else s_bad |= kIlvErrHeader;
      } else {
        s_bad |= kIlvErrHeader;
      }
    }
  }
  __syncthreads();
  // ---- prologue: per coded plane, parse the header and build LDS tables ----
#pragma unroll
  for (uint32_t p = 0; p < NP; ++p) {
    const IlvPlane P = T.planes[p];
    if (!s_slot[p]) continue;
    LutSet& ls = slots[s_slot[p] - 1];
    const uint8_t* pay = reinterpret_cast<const uint8_t*>(P.base);
    build_tables(ls, bs, pay + 5, P.len >= 5 ? P.len - 5 : 0);
    if (t == 0) {
      if (ls.status) s_bad |= kIlvErrHeader;
      uint64_t head = 5 + bs.hdr_len;
      head += (4 - head % 4) % 4;
      const uint64_t data0 = head + 4ull * (nb + 1);
      if (data0 > P.len) {
        s_bad |= kIlvErrHeader;
      } else {
        s_table[p] = P.base + head;
        s_data[p] = P.base + data0;
        s_datalen[p] = P.len - data0;
        const uint32_t* tab = reinterpret_cast<const uint32_t*>(P.base + head);
        if (tab[0] != 0 || tab[nb] != s_datalen[p]) s_bad |= kIlvErrBlock;
      }
    }
    __syncthreads();
  }
  if (s_bad) {
    if (t == 0) atomicOr(&status[tile.tensor], s_bad);
    return;
  }
  // ---- main loop: one wavefront per block ----
  const uint32_t wave = t >> 6, lane = t & 63u;
  uint32_t bad = 0;
  uint8_t* out = reinterpret_cast<uint8_t*>(T.out);
  uint32_t* const sw = word_stage + wave * stage_words;
  for (uint32_t bi = tile.block0 + wave; bi < tile.block0 + tile.nblocks; bi += 4) {
    const uint64_t bstart = (uint64_t)bi * kIlvBlock;
    LaneBits lb[NP];
    LaneLds ll[NP];
    uint32_t lane_c[NP];
    bool staged[NP];
    uint32_t budget = stage_words;
    // the previous block's last reads of `sw` must finish before restaging
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (uint32_t p = 0; p < NP; ++p) {
      lane_c[p] = 0;
      staged[p] = false;
      lb[p].ptr = lb[p].end = lb[p].safe = lb[p].start = nullptr;
      lb[p].buf = 0;
      lb[p].cnt = 0;
      lb[p].nxt = 0;
      ll[p].off = ll[p].end = ll[p].start = ll[p].cnt = ll[p].nxt = 0;
      ll[p].buf = 0;
      if (!s_slot[p]) continue;
      const uint32_t* tab = reinterpret_cast<const uint32_t*>(s_table[p]);
      const uint32_t o0 = tab[bi], o1 = tab[bi + 1];
      const bool bok = o1 >= o0 && o1 <= s_datalen[p] && o1 - o0 >= 64;
      const uint8_t* blk = reinterpret_cast<const uint8_t*>(s_data[p]) + (bok ? o0 : 0);
      const uint32_t c = bok ? blk[lane] : 0u;
      const uint32_t incl = wave_incl_scan(c);
      const uint32_t total = __shfl(incl, 63, 64);
      const bool sized = bok && 64u + 4u * total == o1 - o0;
      if (!sized) bad |= kIlvErrBlock;
      const uint32_t* words = reinterpret_cast<const uint32_t*>(blk + 64);
      lane_c[p] = c;
      if (sized && total <= budget) {
        // coalesced copy of the block's words into this wavefront's LDS
        const uint32_t base = stage_words - budget;
        for (uint32_t i = lane; i < total; i += 64) sw[base + i] = gload_u32(words + i);
        budget -= total;
        staged[p] = true;
        lane_start_lds(ll[p], sw, base + incl - c, base + incl);
      } else {
        lane_start(lb[p], words + (incl - c), sized ? words + incl : words + (incl - c),
                   reinterpret_cast<const uint32_t*>(blk));
      }
    }
    __builtin_amdgcn_wave_barrier();
    for (uint32_t r = 0; r < kIlvRounds; ++r) {
      const uint64_t pos = bstart + (uint64_t)kIlvGroup * (r * 64u + lane);
      const uint32_t count = pos < n ? (uint32_t)(n - pos < kIlvGroup ? n - pos : kIlvGroup) : 0u;
      uint32_t v[NP][4];
#pragma unroll
      for (uint32_t p = 0; p < NP; ++p) {
        const uint64_t raw = s_raw[p] + pos;
        if (staged[p]) {
          decode_group_lds(slots[s_slot[p] - 1], sw, ll[p], count, stage_base + 20u * t, v[p][0], v[p][1], v[p][2],
                           v[p][3]);
        } else if (s_slot[p]) {
          decode_group(slots[s_slot[p] - 1], lb[p], count, stage_base + 20u * t, v[p][0], v[p][1], v[p][2], v[p][3]);
        } else if (count == kIlvGroup && (raw & 15u) == 0) {
          u32x4 x = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(raw));
          v[p][0] = x.x; v[p][1] = x.y; v[p][2] = x.z; v[p][3] = x.w;
        } else {
          uint32_t tmp[4] = {0, 0, 0, 0};
          const uint8_t* src = reinterpret_cast<const uint8_t*>(raw);
          for (uint32_t k = 0; k < count; ++k) tmp[k >> 2] |= (uint32_t)src[k] << (8 * (k & 3));
          v[p][0] = tmp[0]; v[p][1] = tmp[1]; v[p][2] = tmp[2]; v[p][3] = tmp[3];
        }
      }
      if (count == 0) continue;
      uint32_t o[4 * RATIO];
      merge_group<kChain>(v, o);
      if (count == kIlvGroup) {
        u32x4* dst = reinterpret_cast<u32x4*>(out + RATIO * pos);
#pragma unroll
        for (uint32_t k = 0; k < RATIO; ++k)
          __builtin_nontemporal_store(u32x4_make(o[4 * k], o[4 * k + 1], o[4 * k + 2], o[4 * k + 3]), dst + k);
      } else {
        for (uint32_t k = 0; k < RATIO * count; ++k) out[RATIO * pos + k] = (uint8_t)(o[k >> 2] >> (8 * (k & 3)));
      }
    }
    // acceptance: every lane's words hold exactly its codes
#pragma unroll
    for (uint32_t p = 0; p < NP; ++p) {
      if (!s_slot[p]) continue;
      const uint32_t used = staged[p] ? lane_used_lds(ll[p]) : lane_used(lb[p]);
      if ((used + 31u) / 32u != lane_c[p]) bad |= kIlvErrLane;
    }
  }
  if (bad) atomicOr(&status[tile.tensor], bad);
}

// ---------------------------------------------------------------------------
// encode kernels
// ---------------------------------------------------------------------------

__global__ void __launch_bounds__(256) ilv_hist_kernel(const IlvEncPlane* __restrict__ planes,
                                                       uint32_t* __restrict__ hist) {
  __shared__ uint32_t h[4][256];
  const IlvEncPlane P = planes[blockIdx.y];
  const uint32_t t = threadIdx.x, wave = t >> 6;
  for (uint32_t i = t; i < 1024; i += 256) (&h[0][0])[i] = 0;
  __syncthreads();
  const uint8_t* src = reinterpret_cast<const uint8_t*>(P.src);
  const uint64_t nvec = P.n / 16;
  const uint64_t stride = (uint64_t)gridDim.x * 256u;
  for (uint64_t v = (uint64_t)blockIdx.x * 256u + t; v < nvec; v += stride) {
    u32x4 x = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src) + v);
    const uint32_t xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int b = 0; b < 4; ++b) atomicAdd(&h[wave][(xs[k] >> (8 * b)) & 0xFF], 1u);
  }
  if (blockIdx.x == 0)
    for (uint64_t i = nvec * 16 + t; i < P.n; i += 256) atomicAdd(&h[wave][src[i]], 1u);
  __syncthreads();
  uint32_t s = h[0][t] + h[1][t] + h[2][t] + h[3][t];
  if (s) atomicAdd(&hist[256u * blockIdx.y + t], s);
}

// One wavefront per block: lane word counts and block byte size.
__global__ void __launch_bounds__(64) ilv_size_kernel(const IlvEncPlane* __restrict__ planes,
                                                      const IlvEncBlock* __restrict__ blocks,
                                                      const uint32_t* __restrict__ codes,
                                                      uint8_t* __restrict__ lane_words,
                                                      uint32_t* __restrict__ block_bytes) {
  __shared__ uint8_t len[256];
  const IlvEncBlock B = blocks[blockIdx.x];
  const IlvEncPlane P = planes[B.plane];
  const uint32_t lane = threadIdx.x;
  for (uint32_t i = lane; i < 256; i += 64) len[i] = (uint8_t)(codes[256u * P.code_slot + i] >> 16);
  __syncthreads();
  const uint8_t* src = reinterpret_cast<const uint8_t*>(P.src);
  const uint64_t bstart = (uint64_t)B.block * kIlvBlock;
  uint32_t bits = 0;
  for (uint32_t r = 0; r < kIlvRounds; ++r) {
    const uint64_t pos = bstart + (uint64_t)kIlvGroup * (r * 64u + lane);
    if (pos >= P.n) continue;
    if (P.n - pos >= kIlvGroup) {
      u32x4 x = *reinterpret_cast<const u32x4*>(src + pos);
      const uint32_t xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int b = 0; b < 4; ++b) bits += len[(xs[k] >> (8 * b)) & 0xFF];
    } else {
      for (uint64_t k = pos; k < P.n; ++k) bits += len[src[k]];
    }
  }
  const uint32_t words = (bits + 31) / 32;
  lane_words[64ull * blockIdx.x + lane] = (uint8_t)words;
  uint32_t incl = wave_incl_scan(words);
  if (lane == 63) block_bytes[blockIdx.x] = 64u + 4u * incl;
}

// One wavefront per block: write lane word counts and packed lane streams.
__global__ void __launch_bounds__(64) ilv_encode_kernel(const IlvEncPlane* __restrict__ planes,
                                                        const IlvEncBlock* __restrict__ blocks,
                                                        const uint32_t* __restrict__ codes,
                                                        const uint8_t* __restrict__ lane_words) {
  __shared__ uint32_t code[256];
  const IlvEncBlock B = blocks[blockIdx.x];
  const IlvEncPlane P = planes[B.plane];
  const uint32_t lane = threadIdx.x;
  for (uint32_t i = lane; i < 256; i += 64) code[i] = codes[256u * P.code_slot + i];
  __syncthreads();
  uint8_t* blk = reinterpret_cast<uint8_t*>(B.dst);
  const uint32_t c = lane_words[64ull * B.lw + lane];
  blk[lane] = (uint8_t)c;
  const uint32_t incl = wave_incl_scan(c);
  uint32_t* w = reinterpret_cast<uint32_t*>(blk + 64) + (incl - c);
  const uint8_t* src = reinterpret_cast<const uint8_t*>(P.src);
  const uint64_t bstart = (uint64_t)B.block * kIlvBlock;
  uint64_t acc = 0;
  uint32_t cnt = 0, wi = 0;
  for (uint32_t r = 0; r < kIlvRounds; ++r) {
    const uint64_t pos = bstart + (uint64_t)kIlvGroup * (r * 64u + lane);
    if (pos >= P.n) continue;
    const uint64_t end = P.n - pos >= kIlvGroup ? pos + kIlvGroup : P.n;
    for (uint64_t k = pos; k < end; ++k) {
      const uint32_t e = code[src[k]];
      acc |= (uint64_t)(e & 0xFFFFu) << cnt;
      cnt += e >> 16;
      if (cnt >= 32) {
        w[wi++] = (uint32_t)acc;
        acc >>= 32;
        cnt -= 32;
      }
    }
  }
  if (cnt) w[wi++] = (uint32_t)acc;
}

hipError_t launch_ilv_decode(uint32_t chain, const IlvTensor* tensors, const IlvTile* tiles, uint32_t n_tiles,
                             uint32_t* status, uint32_t n_slots, hipStream_t stream) {
  if (!n_tiles) return hipSuccess;
  const dim3 g(n_tiles), b(256);
  // word staging per wavefront: up to 6.5 KB, within a 64 KB workgroup
  // budget, and never smaller than the table-build scratch it aliases
  const size_t fixed = (size_t)n_slots * sizeof(LutSet) + 256 * 20;
  size_t per_wave = (65536 - fixed) / 4;
  if (per_wave > 6656) per_wave = 6656;
  per_wave &= ~(size_t)15;
  if (per_wave * 4 < kIlvScratchBytes) return hipErrorInvalidValue;
  const uint32_t stage_words = (uint32_t)(per_wave / 4);
  const size_t lds = fixed + 4 * per_wave;
  switch (chain) {
#define PTWM_ILV_CASE(C)                                                                              \
  case C:                                                                                             \
    hipLaunchKernelGGL(ilv_decode_kernel<C>, g, b, lds, stream, tensors, tiles, status, n_slots, stage_words); \
    break;
    PTWM_ILV_CASE(kChainIeee16Split2)
    PTWM_ILV_CASE(kChainIeee32Split4)
    PTWM_ILV_CASE(kChainE4m3Nibble)
    PTWM_ILV_CASE(kChainE5m2Nibble)
    PTWM_ILV_CASE(kChainNibbleSplit)
    PTWM_ILV_CASE(kChainPassthrough)
#undef PTWM_ILV_CASE
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_ilv_hist(const IlvEncPlane* planes, uint32_t n_planes, uint64_t max_n, uint32_t* hist,
                           hipStream_t stream) {
  if (!n_planes) return hipSuccess;
  uint64_t blocks = (max_n / 16 + 255) / 256;
  if (blocks > 512) blocks = 512;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(ilv_hist_kernel, dim3((uint32_t)blocks, n_planes), dim3(256), 0, stream, planes, hist);
  return hipGetLastError();
}

hipError_t launch_ilv_size(const IlvEncPlane* planes, const IlvEncBlock* blocks, uint32_t n_blocks,
                           const uint32_t* codes, uint8_t* lane_words, uint32_t* block_bytes, hipStream_t stream) {
  if (!n_blocks) return hipSuccess;
  hipLaunchKernelGGL(ilv_size_kernel, dim3(n_blocks), dim3(64), 0, stream, planes, blocks, codes, lane_words,
                     block_bytes);
  return hipGetLastError();
}

hipError_t launch_ilv_encode(const IlvEncPlane* planes, const IlvEncBlock* blocks, uint32_t n_blocks,
                             const uint32_t* codes, const uint8_t* lane_words, hipStream_t stream) {
  if (!n_blocks) return hipSuccess;
  hipLaunchKernelGGL(ilv_encode_kernel, dim3(n_blocks), dim3(64), 0, stream, planes, blocks, codes, lane_words);
  return hipGetLastError();
}

}  // namespace ptwm
