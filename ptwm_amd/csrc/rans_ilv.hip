// rans_ilv.hip -- the GPU-native interleaved rANS plane codec on gfx950.
//
// Wire format (codec wire id 0x7F02, this library's second plane codec; the
// executable specification is oracle por_rans_ilv_encode/decode):
//   [tag u8] 0: stored plane bytes follow.  2: packed nibbles, as huff_ilv.
//   1: coded:
//   [n u32][max_sym u8][f u16 x (max_sym + 1)][0-pad to 4]
//   [block offset table u32 x (nb + 1)][data],  nb = ceil(n / 16384)
//   frequencies: the reference's normalisation (rans/compress.rs:72-135),
//   11-bit, summing to 2048.
//   block b = [nw u32][x_j u32, j = 0..63][w u16 x nw][0-pad to 4]
//   Lane j owns the 16-symbol groups g = j + 64 r (r = 0..15) of the block,
//   exactly like huff_ilv.  Step s = 16 r + t: every lane whose position
//   16384 b + 16 (64 r + j) + t is inside the plane decodes one symbol
//   (slot = x & 2047, x = f (x >> 11) + slot - cum) and, when x < 2^16,
//   takes the next 16-bit word; the lanes of one step take words in lane
//   order.  Encoding starts every lane at 2^16, so a block is accepted
//   iff all nw words are taken and every final state is 2^16.
//
// Decode: one wavefront per block, persistent workgroups over 4-block tiles
// (as huff_ilv), the plane's 2048-entry slot table (symbol' | f << 8 |
// (slot - cum) << 20, symbol' already through the plane's part of the
// inverse chain) in LDS, the block's words staged in LDS by coalesced
// loads.  A step is one table lookup, one multiply-add, one ballot and one
// LDS word read per lane; the word index is the wavefront's running count
// plus the lane's rank among the lanes that renormalise (mbcnt).  Rounds
// end in the same merge and dwordx4 stores as huff_ilv.
//
// Encode: histogram (shared with huff_ilv), host normalisation, a size pass
// (one wavefront per block runs the encoder and counts words), host layout,
// and a write pass that runs the encoder again and writes each step's words
// below the previous step's (the decoder reads the stream forward).
#include "rans_ilv.h"

#include "ilv_common.h"

namespace ptwm {

namespace {


struct alignas(16) RilvCtl {
  uint64_t table[4];    // per plane: block offset table address
  uint64_t data[4];     // block data base
  uint64_t datalen[4];  // block data bytes
  uint64_t raw[4];      // stored plane bytes (tag 0 or raw planes)
  uint32_t coded[4];
  uint32_t packed[4];   // plane stored as packed nibbles (tag 2)
  uint32_t slot[4];     // LDS table slot of a coded plane
  uint32_t bad;
  uint32_t wsum[4];     // table build scratch: per-wavefront frequency sums
  uint32_t last[4];     // last byte of each native payload
  uint32_t pad[3];
  uint16_t cum[264];    // table build scratch: cumulative frequencies
  uint16_t f[256];
};
static_assert(sizeof(RilvCtl) % 16 == 0, "RilvCtl keeps the staging area 16-byte aligned");

__device__ __forceinline__ uint32_t ld_le32(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// One step of one coded plane for the wavefront.  lut: LDS address of the
// plane's table; the block's nw words are staged at LDS byte address sw or
// read from global memory at gw; wpos: words taken so far (uniform).  Word
// indexes are clamped to the block and a block without words reads none,
// so malformed input only fails acceptance.
template <bool kTail, bool kStaged>
__device__ __forceinline__ uint32_t rilv_step(uint32_t& x, uint32_t lut, uint32_t sw, uint64_t gw, uint32_t nw,
                                              uint32_t& wpos, bool active) {
  const uint32_t slot = x & 2047u;
  const uint32_t e = lds_ld32(lut + 4u * slot);
  const uint32_t xd = ((e >> 8) & 0xFFFu) * (x >> kRilvProbBits) + (e >> 20);
  const bool need = (!kTail || active) && xd < kRilvL;
  const uint64_t bal = __ballot(need);
  const uint32_t rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
  uint32_t wi = wpos + rank;
  wi = wi < nw ? wi : (nw ? nw - 1 : 0);
  uint32_t w = 0;
  if constexpr (kStaged) {
    w = lds_ld16(sw + 2u * wi);
  } else {
    if (need && nw) w = g_ld<uint16_t>(gw + 2ull * wi);
  }
  if (!kTail || active) x = need ? (xd << 16) | w : xd;
  wpos += (uint32_t)__builtin_popcountll(bal);
  return (!kTail || active) ? (e & 0xFFu) : 0u;
}

struct RilvBlock {
  uint32_t x[4];      // lane state per plane
  uint32_t sw[4];     // staged words: LDS byte address
  uint64_t gw[4];     // words in global memory
  uint32_t wpos[4];   // words taken
  uint32_t nw[4];
  uint64_t raw[4];
  uint32_t rbytes[4];  // bytes of a raw plane's data (0 for a coded plane)
  uint32_t lut[4];     // LDS address of a coded plane's table
  uint32_t coded_mask;
  uint32_t packed_mask;
};

template <uint32_t kChain, bool kTail, bool kStaged>
__device__ __forceinline__ void rilv_decode_block(RilvBlock& st, uint32_t luts, uint64_t out, uint64_t n,
                                                  uint64_t bstart, uint32_t lane) {
  constexpr uint32_t NP = ChainInfo<kChain>::np;
  constexpr uint32_t RATIO = ChainInfo<kChain>::ratio;
  // full blocks: the raw planes' next group is loaded a round ahead, one
  // buffer load per plane (see load_group_fast), so its latency overlaps
  // the round's rANS steps
  uint32_t nxt[NP][4];
  if constexpr (!kTail) {
#pragma unroll
    for (uint32_t p = 0; p < NP; ++p)
      load_group_fast(st.raw[p], st.rbytes[p], (st.packed_mask >> p) & 1u, (uint32_t)(bstart + kIlvGroup * lane), true,
                      nxt[p]);
#pragma unroll
    for (uint32_t k = 0; k < RATIO; ++k) vmem_nop(out, k);
  }
  for (uint32_t r = 0; r < kIlvRounds; ++r) {
    const uint64_t pos = bstart + (uint64_t)kIlvGroup * (r * 64u + lane);
    const uint32_t count = group_count<kTail>(pos, n);
    uint32_t v[NP][4];
#pragma unroll
    for (uint32_t p = 0; p < NP; ++p) {
      v[p][0] = v[p][1] = v[p][2] = v[p][3] = 0;
      if constexpr (kTail) {
        if (st.coded_mask & (1u << p)) continue;
        // stored plane: the group's 16 bytes (or 8 bytes of packed nibbles)
        load_group(st.raw[p], (st.packed_mask >> p) & 1u, pos, count, v[p]);
#pragma unroll
        for (int k = 0; k < 4; ++k) v[p][k] = xform_word(ChainInfo<kChain>::xf[p], v[p][k]);
      } else {
        // every plane's load is consumed here (coded planes loaded zeros)
        uint32_t x[4];
        expand_group((st.packed_mask >> p) & 1u, nxt[p], x);
        const bool raw = !(st.coded_mask & (1u << p));
#pragma unroll
        for (int k = 0; k < 4; ++k) v[p][k] = raw ? xform_word(ChainInfo<kChain>::xf[p], x[k]) : 0u;
      }
    }
    if constexpr (!kTail) {
#pragma unroll
      for (uint32_t p = 0; p < NP; ++p)
        load_group_fast(st.raw[p], st.rbytes[p], (st.packed_mask >> p) & 1u, (uint32_t)(pos + kIlvGroup * 64u),
                        r + 1 < kIlvRounds, nxt[p]);
    }
#pragma unroll
    for (uint32_t t = 0; t < kIlvGroup; ++t) {
      const bool active = t < count;
#pragma unroll
      for (uint32_t p = 0; p < NP; ++p) {
        if (!(st.coded_mask & (1u << p))) continue;
        const uint32_t lut = st.lut[p];
        const uint32_t sym = rilv_step<kTail, kStaged>(st.x[p], lut, st.sw[p], st.gw[p], st.nw[p], st.wpos[p], active);
        v[p][t >> 2] |= sym << (8 * (t & 3));
      }
    }
    if (kTail && count == 0) continue;
    uint32_t o[4 * RATIO];
    merge_group<kChain>(v, o);
    const uint64_t dst = out + RATIO * pos;
    if constexpr (!kTail) {
      store_group_full<RATIO>(dst, lane, o);
    } else if (count == kIlvGroup) {
#pragma unroll
      for (uint32_t k = 0; k < RATIO; ++k)
        g_st<u32x4>(dst + 16 * k, u32x4_make(o[4 * k], o[4 * k + 1], o[4 * k + 2], o[4 * k + 3]));
    } else {
      for (uint32_t k = 0; k < RATIO * count; ++k) gstore_u8(dst + k, o[k >> 2] >> (8 * (k & 3)));
    }
  }
}

// Build plane p's slot table at LDS table `tab` from the payload's
// frequency header (all threads; ctl.f / ctl.cum filled by thread 0).
template <uint32_t kChain>
__device__ __forceinline__ void rilv_build_table(uint32_t* tab, const RilvCtl& ctl, uint32_t xf) {
  for (uint32_t slot = threadIdx.x; slot < 2048u; slot += blockDim.x) {
    // the symbol s with cum[s] <= slot < cum[s + 1] (cum[256] = 2048)
    uint32_t lo = 0, hi = 256;
    while (hi - lo > 1) {
      const uint32_t mid = (lo + hi) >> 1;
      if (ctl.cum[mid] <= slot) lo = mid;
      else hi = mid;
    }
    tab[slot] = xform_byte(xf, lo) | ((uint32_t)ctl.f[lo] << 8) | ((slot - ctl.cum[lo]) << 20);
  }
}

template <uint32_t kChain>
__global__ void __launch_bounds__(256) rilv_decode_kernel(const IlvTensor* __restrict__ tensors,
                                                          const uint32_t* __restrict__ tix,
                                                          const uint32_t* __restrict__ tpre, uint32_t m,
                                                          uint32_t* __restrict__ status, uint32_t n_slots,
                                                          uint32_t stage_words) {
  constexpr uint32_t NP = ChainInfo<kChain>::np;
  // LDS: [n_slots tables (coded planes from the last one down)][RilvCtl][4 x stage_words]
  extern __shared__ __align__(16) uint8_t smem[];
  RilvCtl& ctl = *reinterpret_cast<RilvCtl*>(smem + n_slots * kRilvTableBytes);
  uint32_t* const stage = reinterpret_cast<uint32_t*>(smem + n_slots * kRilvTableBytes + sizeof(RilvCtl));
  // while a tensor's tables are built, the staging area holds the payload
  // heads (the host sizes it for NP x kRilvHeadWords words at least)
  uint32_t (*const head)[kRilvHeadWords] = reinterpret_cast<uint32_t (*)[kRilvHeadWords]>(stage);
  const uint32_t luts = lds_addr(smem);
  const uint32_t t = threadIdx.x, wave = t >> 6, lane = t & 63u;
  const uint32_t n_tiles = tpre[m];
  const uint32_t tile0 = (uint32_t)((uint64_t)blockIdx.x * n_tiles / gridDim.x);
  const uint32_t tile1 = (uint32_t)((uint64_t)(blockIdx.x + 1) * n_tiles / gridDim.x);
  if (tile0 >= tile1) return;
  uint32_t lo = 0, hi = m;
  while (hi - lo > 1) {
    const uint32_t mid = (lo + hi) / 2;
    if (tpre[mid] <= tile0) lo = mid;
    else hi = mid;
  }
  uint32_t j = lo, cur = 0xFFFFFFFFu, bad = 0;
  uint32_t* const sw = stage + wave * stage_words;
  for (uint32_t tile = tile0; tile < tile1; ++tile) {
    while (tile >= tpre[j + 1]) ++j;
    const uint32_t ti = tix[j];
    const IlvTensor& T = tensors[ti];
    const uint64_t n = T.n;
    const uint32_t nb = (uint32_t)((n + kIlvBlock - 1) / kIlvBlock);
    if (ti != cur) {
      // ---- new tensor: parse the plane headers, build the slot tables ----
      bad = wave_or_status(bad);
      if (bad && lane == 0) status_or(&status[cur], bad);
      bad = 0;
      cur = ti;
      __syncthreads();
      // the payload heads and last bytes, loaded by all threads at once
      // (native payloads start 4-byte aligned)
      for (uint32_t k = t; k < NP * (kRilvHeadWords + 1); k += 256) {
        const uint32_t p = k / (kRilvHeadWords + 1), w = k % (kRilvHeadWords + 1);
        const uint64_t base = T.planes[p].base, len = T.planes[p].len;
        uint32_t v = 0;
        if (T.planes[p].coded) {
          if (w == kRilvHeadWords) {
            if (len) v = gload_u8(base + len - 1);
          } else if (4ull * w + 4 <= len) {
            v = g_ld<uint32_t>(base + 4ull * w);
          } else {
            for (uint64_t b = 4ull * w; b < len && b < 4ull * w + 4; ++b) v |= gload_u8(base + b) << (8 * (b & 3));
          }
        }
        if (w == kRilvHeadWords) ctl.last[p] = v;
        else head[p][w] = v;
      }
      __syncthreads();
      if (t == 0) {
        ctl.bad = 0;
        for (uint32_t p = 0; p < NP; ++p) {
          const IlvPlane& P = T.planes[p];
          ctl.raw[p] = P.base;
          ctl.coded[p] = 0;
          ctl.packed[p] = 0;
          if (!P.coded) continue;
          const uint8_t* pay = reinterpret_cast<const uint8_t*>(head[p]);
          if (P.len == 0) ctl.bad |= kIlvErrHeader;
          else if (pay[0] == 0) {
            if (P.len != n + 1) ctl.bad |= kIlvErrHeader;
            ctl.raw[p] = P.base + 1;
          } else if (pay[0] == 2) {
            if (!packed_header_ok(pay, P.len, n, ctl.last[p])) ctl.bad |= kIlvErrHeader;
            ctl.raw[p] = P.base + kPackedHeadBytes;
            ctl.packed[p] = 1;
          } else if (pay[0] == 1 && P.len >= 6 && ld_le32(pay + 1) == n) {
            ctl.coded[p] = 1;
          } else {
            ctl.bad |= kIlvErrHeader;
          }
        }
        // table slots of the coded planes, from the last plane down
        uint32_t k = 0;
        for (uint32_t p = NP; p-- > 0;) {
          ctl.slot[p] = k;
          if (!ctl.coded[p]) continue;
          if (k < n_slots) {
            ++k;
          } else {  // no table for it in this launch: the tensor is decoded again
            ctl.coded[p] = 0;
            ctl.bad |= kIlvRetrySlots;
          }
        }
      }
      __syncthreads();
#pragma unroll
      for (uint32_t p = 0; p < NP; ++p) {
        if (!ctl.coded[p]) continue;
        const IlvPlane P = T.planes[p];
        const uint8_t* pay = reinterpret_cast<const uint8_t*>(head[p]);
        // frequencies: f[s] for s <= max_sym, cumulative by a workgroup scan
        const uint32_t ms = pay[5];
        const uint64_t hl = 6 + 2ull * (ms + 1);
        const bool hok = hl <= P.len;  // the head holds 6 + 512 bytes at most
        const uint32_t fs = hok && t <= ms ? (uint32_t)pay[6 + 2 * t] | ((uint32_t)pay[7 + 2 * t] << 8) : 0u;
        const uint32_t incl = wave_incl_scan(fs);
        if (lane == 63) ctl.wsum[wave] = incl;
        __syncthreads();
        uint32_t run = incl - fs;
        for (uint32_t wv = 0; wv < wave; ++wv) run += ctl.wsum[wv];
        ctl.cum[t] = (uint16_t)(run < 2048u ? run : 2048u);
        ctl.f[t] = (uint16_t)fs;
        if (t == 0) {
          ctl.cum[256] = 2048;
          const uint32_t total = ctl.wsum[0] + ctl.wsum[1] + ctl.wsum[2] + ctl.wsum[3];
          bool ok = hok && total == 2048u;
          const uint64_t head = (hl + 3) & ~3ull;
          const uint64_t data0 = head + 4ull * (nb + 1);
          ok = ok && data0 <= P.len;
          for (uint64_t i = hl; ok && i < head; ++i)
            if (pay[i]) ok = false;
          if (!ok) {
            ctl.bad |= kIlvErrHeader;
          } else {
            // tab[0] == 0 and tab[nb] == datalen are checked by the
            // wavefronts of the first and last block
            ctl.table[p] = P.base + head;
            ctl.data[p] = P.base + data0;
            ctl.datalen[p] = P.len - data0;
          }
        }
        __syncthreads();
        if (!ctl.bad)
          rilv_build_table<kChain>(reinterpret_cast<uint32_t*>(smem + ctl.slot[p] * kRilvTableBytes), ctl,
                                   ChainInfo<kChain>::xf[p]);
        __syncthreads();
      }
      if (t == 0 && ctl.bad) status_or(&status[ti], ctl.bad);
    }
    if (ctl.bad) continue;  // uniform: the tensor is rejected
    const uint32_t bi = kIlvBlocksPerTile * (tile - tpre[j]) + wave;
    if (bi >= nb) continue;
    // ---- one wavefront per block ----
    const uint64_t bstart = (uint64_t)bi * kIlvBlock;
    RilvBlock st;
    st.coded_mask = 0;
    st.packed_mask = 0;
    bool ok = true;
    uint32_t need = 0;
    uint64_t wsrc[4];
#pragma unroll
    for (uint32_t p = 0; p < NP; ++p) {
      st.raw[p] = ctl.raw[p];
      st.lut[p] = luts + __builtin_amdgcn_readfirstlane(ctl.slot[p]) * kRilvTableBytes;
      if (__builtin_amdgcn_readfirstlane(ctl.packed[p])) st.packed_mask |= 1u << p;
      st.x[p] = kRilvL;
      st.sw[p] = 0;
      st.gw[p] = 0;
      st.wpos[p] = 0;
      st.nw[p] = 0;
      wsrc[p] = 0;
      if (!__builtin_amdgcn_readfirstlane(ctl.coded[p])) continue;
      st.coded_mask |= 1u << p;
      const uint64_t tb = ctl.table[p];
      const uint32_t o0 = g_ld<uint32_t>(tb + 4ull * bi), o1 = g_ld<uint32_t>(tb + 4ull * bi + 4);
      const bool bok = o1 >= o0 && o1 - o0 >= kRilvBlockHead && o1 <= ctl.datalen[p] && (o0 & 3u) == 0 &&
                       (bi != 0 || o0 == 0) && (bi + 1 != nb || o1 == ctl.datalen[p]);
      const uint64_t blk = ctl.data[p] + (bok ? o0 : 0);
      const uint32_t nwb = bok ? g_ld<uint32_t>(blk) : 0u;
      if (!bok || nwb > 16384u || ((kRilvBlockHead + 2u * nwb + 3u) & ~3u) != o1 - o0) ok = false;
      else if ((nwb & 1u) && g_ld<uint16_t>(blk + kRilvBlockHead + 2ull * nwb) != 0) ok = false;
      if (!ok) break;
      st.x[p] = g_ld<uint32_t>(blk + 4 + 4 * lane);
      st.nw[p] = nwb;
      wsrc[p] = blk + kRilvBlockHead;
      st.gw[p] = wsrc[p];
      need += ((nwb + 1) / 2 + 3u) & ~3u;
    }
    if (!ok) {
      bad |= kIlvErrBlock;
      continue;
    }
    // the fast path takes whole blocks of planes under 4 GiB whose raw
    // planes are aligned
    bool full = bstart + kIlvBlock <= n && n <= 0xFFFFFFFFull;
#pragma unroll
    for (uint32_t p = 0; p < NP; ++p) {
      const bool packed = (st.packed_mask >> p) & 1u;
      st.rbytes[p] = (st.coded_mask & (1u << p)) ? 0u : (uint32_t)(packed ? (n + 1) / 2 : n);
      if (!(st.coded_mask & (1u << p)) && !raw_aligned(st.raw[p], packed)) full = false;
    }
    const uint64_t out = T.out;
    if (need <= stage_words) {
      // coalesced copy of each coded plane's words into this wavefront's LDS
      __builtin_amdgcn_wave_barrier();
      uint32_t base = 0;
#pragma unroll
      for (uint32_t p = 0; p < NP; ++p) {
        if (!(st.coded_mask & (1u << p))) continue;
        const uint32_t nd = (st.nw[p] + 1) / 2;
        for (uint32_t i = lane; i < nd; i += 64) sw[base + i] = g_ld<uint32_t>(wsrc[p] + 4ull * i);
        st.sw[p] = lds_addr(sw + base);
        base += (nd + 3u) & ~3u;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if (full) rilv_decode_block<kChain, false, true>(st, luts, out, n, bstart, lane);
      else rilv_decode_block<kChain, true, true>(st, luts, out, n, bstart, lane);
      __builtin_amdgcn_wave_barrier();
    } else {
      rilv_decode_block<kChain, true, false>(st, luts, out, n, bstart, lane);
    }
    // acceptance: every word taken, every lane back at 2^16
#pragma unroll
    for (uint32_t p = 0; p < NP; ++p) {
      if (!(st.coded_mask & (1u << p))) continue;
      if (st.wpos[p] != st.nw[p] || __ballot(st.x[p] != kRilvL) != 0) bad |= kRilvErrState;
    }
  }
  bad = wave_or_status(bad);
  if (bad && lane == 0) status_or(&status[cur], bad);
}

// ---------------------------------------------------------------------------
// encode
// ---------------------------------------------------------------------------

// Symbol of step s for lane `lane` of block `b` (position pos) and whether
// it is inside the plane.
__device__ __forceinline__ uint64_t rilv_pos(uint32_t b, uint32_t lane, uint32_t s) {
  return (uint64_t)b * kIlvBlock + (uint64_t)kIlvGroup * (64u * (s / kIlvGroup) + lane) + (s % kIlvGroup);
}

// 1 / f of each symbol's frequency (f = 0, a symbol the histogram did not
// see, as 1), for the encoder's quotient estimate
__device__ __forceinline__ float rilv_rcp(uint32_t fc) {
  const uint32_t f0 = fc & 0xFFFFu;
  return 1.0f / (float)(f0 ? f0 : 1u);
}

// The encoder's step for one lane: renormalise (emit) then encode.  After
// renormalisation x < f 2^21, so q = x / f < 2^21 and the float estimate
// x * (1 / f) is within one of it (x rounds by at most f / 8, the product
// and the reciprocal add under 2^-22 relative); one correction step makes
// q and r exact.
__device__ __forceinline__ bool rilv_enc_step(uint32_t& x, uint32_t fc, float rf, uint32_t& word) {
  const uint32_t f0 = fc & 0xFFFFu, c = fc >> 16;
  const uint32_t f = f0 ? f0 : 1u;  // a symbol the histogram did not see (source changed): a bad stream, no trap
  const bool emit = (uint64_t)x >= ((uint64_t)f << 21);
  word = x & 0xFFFFu;
  if (emit) x >>= 16;
  uint32_t q = (uint32_t)((float)x * rf);
  int32_t r = (int32_t)(x - q * f);  // true value in [-f, 2f): exact as int32
  if (r < 0) {
    --q;
    r += (int32_t)f;
  } else if (r >= (int32_t)f) {
    ++q;
    r -= (int32_t)f;
  }
  x = q * 2048u + (uint32_t)r + c;
  return emit;
}

// The 16 plane bytes of the group starting at position g0 (zero past the end).
__device__ __forceinline__ void rilv_load_group(const IlvEncPlane& P, uint64_t g0, uint32_t (&sym)[4]) {
  sym[0] = sym[1] = sym[2] = sym[3] = 0;
  if (g0 + kIlvGroup <= P.n) {
    const u32x4 v = gload_nt16(P.src + g0);  // planes are 16-byte aligned, groups 16-byte strided
    sym[0] = v.x;
    sym[1] = v.y;
    sym[2] = v.z;
    sym[3] = v.w;
  } else {
    for (uint64_t k = g0; k < P.n; ++k) sym[(k - g0) >> 2] |= gload_u8(P.src + k) << (8 * ((k - g0) & 3));
  }
}

// One wavefront per block: run the encoder and count the words.
__global__ void __launch_bounds__(64) rilv_size_kernel(const IlvEncPlane* __restrict__ planes,
                                                       const RilvEncBlock* __restrict__ blocks,
                                                       const uint32_t* __restrict__ syms,
                                                       uint32_t* __restrict__ block_words) {
  __shared__ uint32_t fc[256];
  __shared__ float rf[256];
  const RilvEncBlock B = blocks[blockIdx.x];
  const IlvEncPlane P = planes[B.plane];
  const uint32_t lane = threadIdx.x;
  for (uint32_t i = lane; i < 256; i += 64) {
    fc[i] = syms[256u * P.code_slot + i];
    rf[i] = rilv_rcp(fc[i]);
  }
  __syncthreads();
  uint32_t x = kRilvL, nw = 0;
  for (int r = (int)kIlvRounds - 1; r >= 0; --r) {
    const uint64_t g0 = rilv_pos(B.block, lane, 16u * (uint32_t)r);
    uint32_t sym[4];
    rilv_load_group(P, g0, sym);
    for (int tt = (int)kIlvGroup - 1; tt >= 0; --tt) {
      bool emit = false;
      if (g0 + tt < P.n) {
        uint32_t w;
        const uint32_t sy = (sym[tt >> 2] >> (8 * (tt & 3))) & 0xFFu;
        emit = rilv_enc_step(x, fc[sy], rf[sy], w);
      }
      nw += (uint32_t)__builtin_popcountll(__ballot(emit));
    }
  }
  if (lane == 0) block_words[blockIdx.x] = nw;
}

// One wavefront per block: run the encoder again and write the block.
__global__ void __launch_bounds__(64) rilv_encode_kernel(const IlvEncPlane* __restrict__ planes,
                                                         const RilvEncBlock* __restrict__ blocks,
                                                         const uint32_t* __restrict__ syms,
                                                         const uint32_t* __restrict__ block_words) {
  __shared__ uint32_t fc[256];
  __shared__ float rf[256];
  const RilvEncBlock B = blocks[blockIdx.x];
  const IlvEncPlane P = planes[B.plane];
  const uint32_t lane = threadIdx.x;
  for (uint32_t i = lane; i < 256; i += 64) {
    fc[i] = syms[256u * P.code_slot + i];
    rf[i] = rilv_rcp(fc[i]);
  }
  __syncthreads();
  const uint32_t nw = block_words[blockIdx.x];
  const uint64_t words = B.dst + kRilvBlockHead;
  uint32_t x = kRilvL, tail = nw;
  for (int r = (int)kIlvRounds - 1; r >= 0; --r) {
    const uint64_t g0 = rilv_pos(B.block, lane, 16u * (uint32_t)r);
    uint32_t sym[4];
    rilv_load_group(P, g0, sym);
    for (int tt = (int)kIlvGroup - 1; tt >= 0; --tt) {
      bool emit = false;
      uint32_t w = 0;
      if (g0 + tt < P.n) {
        const uint32_t sy = (sym[tt >> 2] >> (8 * (tt & 3))) & 0xFFu;
        emit = rilv_enc_step(x, fc[sy], rf[sy], w);
      }
      const uint64_t bal = __ballot(emit);
      tail -= (uint32_t)__builtin_popcountll(bal);
      const uint32_t rank =
          __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
      // (the size pass counted the same words; the bound only guards a
      // source that changed between the passes)
      if (emit && tail + rank < nw) g_st<uint16_t>(words + 2ull * (tail + rank), (uint16_t)w);
    }
  }
  g_st<uint32_t>(B.dst + 4 + 4 * lane, x);
  if (lane == 0) {
    g_st<uint32_t>(B.dst, nw);
    if (nw & 1u) g_st<uint16_t>(words + 2ull * nw, 0);
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

static const void* rilv_decode_fn(uint32_t chain) {
  switch (chain) {
    case kChainIeee16Split2: return reinterpret_cast<const void*>(&rilv_decode_kernel<kChainIeee16Split2>);
    case kChainIeee32Split4: return reinterpret_cast<const void*>(&rilv_decode_kernel<kChainIeee32Split4>);
    case kChainE4m3Nibble: return reinterpret_cast<const void*>(&rilv_decode_kernel<kChainE4m3Nibble>);
    case kChainE5m2Nibble: return reinterpret_cast<const void*>(&rilv_decode_kernel<kChainE5m2Nibble>);
    case kChainNibbleSplit: return reinterpret_cast<const void*>(&rilv_decode_kernel<kChainNibbleSplit>);
    case kChainPassthrough: return reinterpret_cast<const void*>(&rilv_decode_kernel<kChainPassthrough>);
    default: return nullptr;
  }
}

size_t rilv_decode_lds_bytes(uint32_t chain, uint32_t n_slots, uint32_t stage_words) {
  (void)chain;
  return (size_t)n_slots * kRilvTableBytes + sizeof(RilvCtl) + 4ull * stage_words * 4ull;
}

hipError_t rilv_decode_occupancy(uint32_t chain, uint32_t n_slots, uint32_t stage_words, int* wg_per_cu) {
  const void* fn = rilv_decode_fn(chain);
  if (!fn) return hipErrorInvalidValue;
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(wg_per_cu, fn, 256,
                                                      rilv_decode_lds_bytes(chain, n_slots, stage_words));
}

hipError_t launch_rilv_decode(uint32_t chain, const IlvTensor* tensors, const uint32_t* tix, const uint32_t* tpre,
                              uint32_t m, uint32_t grid, uint32_t* status, uint32_t n_slots, uint32_t stage_words,
                              hipStream_t stream) {
  if (m == 0 || grid == 0) return hipSuccess;
  if (stage_words % 4 != 0 || n_slots > 4) return hipErrorInvalidValue;
  const size_t lds = rilv_decode_lds_bytes(chain, n_slots, stage_words);
  if (lds > kRilvMaxLds) return hipErrorInvalidValue;
  switch (chain) {
#define PTWM_RILV_CASE(C)                                                                                      \
  case C:                                                                                                      \
    hipLaunchKernelGGL(rilv_decode_kernel<C>, dim3(grid), dim3(256), lds, stream, tensors, tix, tpre, m, status, \
                       n_slots, stage_words);                                                                  \
    break;
    PTWM_RILV_CASE(kChainIeee16Split2)
    PTWM_RILV_CASE(kChainIeee32Split4)
    PTWM_RILV_CASE(kChainE4m3Nibble)
    PTWM_RILV_CASE(kChainE5m2Nibble)
    PTWM_RILV_CASE(kChainNibbleSplit)
    PTWM_RILV_CASE(kChainPassthrough)
#undef PTWM_RILV_CASE
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_rilv_size(const IlvEncPlane* planes, const RilvEncBlock* blocks, uint32_t n_blocks,
                            const uint32_t* syms, uint32_t* block_words, hipStream_t stream) {
  if (n_blocks == 0) return hipSuccess;
  hipLaunchKernelGGL(rilv_size_kernel, dim3(n_blocks), dim3(64), 0, stream, planes, blocks, syms, block_words);
  return hipGetLastError();
}

hipError_t launch_rilv_encode(const IlvEncPlane* planes, const RilvEncBlock* blocks, uint32_t n_blocks,
                              const uint32_t* syms, const uint32_t* block_words, hipStream_t stream) {
  if (n_blocks == 0) return hipSuccess;
  hipLaunchKernelGGL(rilv_encode_kernel, dim3(n_blocks), dim3(64), 0, stream, planes, blocks, syms, block_words);
  return hipGetLastError();
}

}  // namespace ptwm
