// huff_ilv.hip -- the GPU-native interleaved Huffman plane codec on gfx950.
//
// Wire format (codec wire id 0x7F01, this library's plane-codec id):
//   [tag u8] 0: stored plane bytes follow.  2: packed nibbles,
//   [n u32][0 0 0][ceil(n / 2) bytes], byte i = s[2i] | s[2i+1] << 4 (a plane
//   of symbols < 16 that codes no smaller, e.g. MXFP4 codes).  1: coded:
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
// of a round is one contiguous span: all stores are coalesced dwordx4.  The
// block's lane streams are first copied into the wavefront's LDS region with
// coalesced loads; every lane then decodes its 16 symbols per round on a
// fixed schedule (no data-dependent branches): every second symbol a 32-bit
// window is read from LDS at the lane's bit position (ds_read2 + alignbit)
// and two 11-bit table lookups consume it.  The 2048-entry table (one entry
// per 11-bit window) is built per workgroup in LDS from the payload's
// weights header.  Tensors whose planes are all stored-aligned or
// huff_ilv-coded are decoded and merged in one pass (decode -> inverse chain
// -> store), so planes never round-trip through HBM.  Workgroups are
// persistent: each takes a contiguous range of 4-block tiles and rebuilds
// its tables only when the range crosses into the next tensor.
//
// Encode: LDS-privatised histograms merged with atomics, host code-table
// build (256 symbols), a size pass (one wave per block: per-lane bit counts
// from the code lengths), a host prefix sum for block offsets, and an encode
// pass that writes each lane's words at its prefix-summed offset.
#include "huff_ilv.h"
#include "crc_device.h"
#include "ilv_common.h"

#include <cstring>

namespace ptwm {

namespace {

// Constant address space: read-only global memory (and the kernel argument
// segment); uniform loads through it become scalar loads.
#define KConst __attribute__((address_space(4)))

__device__ __forceinline__ uint32_t ld_u32le(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// Per-coded-plane decode tables, resident in LDS.
//
// Single mode (any alphabet): 2048 u16 entries, one per 11-bit window,
// entry = code length | symbol' << 8.  Windows that match no code decode as
// symbol 0 with length max_bits (the gap fill of tree.rs:143-169); a table
// for max_bits < 11 is replicated over the unused high index bits.  symbol'
// is the symbol after the plane's part of the inverse chain (Xform),
// so the merge only combines planes.
//
// Pair mode (symbols < 16 and every code <= 6 bits, the huff_ilv encoder's
// choice for nibble planes): 4096 u16 entries, one per 12-bit window,
// each decoding the next two codes: entry = (len0 + len1) | s0 << 8 |
// s1 << 12 (raw nibbles; both codes always fit 12 bits).  Partial groups
// use a 64-entry single-mode table (6-bit windows, symbol' bytes) kept in
// DecodeCtl.
//
// A table slot is 4 KiB for the IEEE and passthrough chains and 8 KiB for
// the nibble chains (the only ones that use pair mode).
constexpr uint32_t kIlvLutBytes = 4096;
constexpr uint32_t kIlvPairLutBytes = 8192;

// Build-time scratch, shared by every plane of the workgroup.
struct BuildScratch {
  uint16_t t64raw[64];  // pair mode: 6-bit single table with raw symbols
  uint8_t sorted[256];  // symbols by (code length, symbol): canonical code order
  uint32_t wave_len_count[4][12];  // per wavefront: symbols of each length ([0]: any length > 11)
  uint32_t cnt[12];                // symbols of each length
  uint32_t off[12];                // per length: canonical index of its first symbol
  uint32_t base[12];               // per length: first canonical index minus first code
  uint32_t lim[12];                // per length: end of the codes of length <= l, left-aligned to 11 bits
  uint32_t err, hdr_len, pair, max_bits;
};

struct alignas(16) DecodeCtl {
  uint16_t t64[4][64];  // pair-mode planes: 6-bit single tables (symbol')
  uint32_t last[4];     // last byte of each native payload
  BuildScratch bs;
  uint64_t table[4], data[4], datalen[4], raw[4];  // per plane
  uint32_t coded[4];
  uint32_t pair[4];
  uint32_t packed[4];   // plane stored as packed nibbles (tag 2)
  uint32_t slot[4];     // LDS table slot of a coded plane
  uint32_t hdr_avail[4];  // bytes of a coded plane's weights header in its head
  uint64_t pbase[4], plen[4];  // the tensor's plane descriptors (IlvPlane)
  uint32_t pcoded[4];
  uint32_t bad;
  uint32_t pad[3];
};
static_assert(sizeof(DecodeCtl) % 16 == 0, "DecodeCtl keeps the staging area 16-byte aligned");

// Layout of a huff_ilv coded payload (tag 1): tag, n (4 bytes), the
// weights header (0x80 | count, or 0x80 then count; then the 4-bit weights),
// padding to 4 bytes, the block offset table (nb + 1 words), the blocks.
// From the payload head `pay` (`avail` valid bytes) sets the table and data
// offsets; false when the header's count bytes are invalid or the table
// does not fit the payload's `len` bytes.
__device__ __forceinline__ bool coded_layout(const uint8_t* pay, uint32_t avail, uint64_t len, uint32_t nb,
                                             uint64_t& table, uint64_t& data) {
  const uint32_t h0 = avail >= 6 ? pay[5] : 0u;
  uint32_t hb = 0, nsym = 0;
  if (h0 & 0x80u) {
    if (h0 != 0x80u) {
      hb = 1;
      nsym = h0 & 0x7Fu;
    } else if (avail >= 7) {
      hb = 2;
      nsym = pay[6] ? pay[6] : 256u;
    }
  }
  uint64_t hd = 5 + hb + (nsym + 1) / 2;
  hd += (4 - hd % 4) % 4;
  table = hd;
  data = hd + 4ull * (nb + 1);
  return hb != 0 && data <= len;
}

// Build the tables of one plane from the weights header at hdr (LDS,
// hdr_avail bytes valid), symbols transformed by `xf`: the pair table at
// `tab` plus the 6-bit table at `t64` when pair_ok and the code allows it,
// else the single table at `tab`.  All 256 threads of the workgroup take
// part: every thread evaluates the header and the per-length counts
// (uniform values), and every table entry is filled by decoding its window
// against the canonical limits: with codes assigned in (length, symbol)
// order, the codes of length <= l, left-aligned to 11 bits, are exactly the
// values below lim[l], so a window's code length is 1 + the number of
// limits it reaches and its symbol is sorted[base[len] + code].  Sets
// bs.err (nonzero: invalid header), bs.pair and bs.hdr_len.
__device__ __forceinline__ void build_tables(uint16_t* tab, uint16_t* t64, bool pair_ok, uint32_t xf, BuildScratch& bs,
                             const uint8_t* hdr, uint64_t hdr_avail) {
  const uint32_t t = threadIdx.x, wave = t >> 6, lane = t & 63u;
  // weights header (weights.rs): 0x80 | n, or 0x80, n (n = 128..256)
  uint32_t err = 0, n = 0, hb = 0;
  const uint32_t h0 = hdr_avail >= 1 ? hdr[0] : 0u;
  if (!(h0 & 0x80u)) {
    err = 1;
  } else if (h0 == 0x80u) {
    if (hdr_avail < 2) {
      err = 1;
    } else {
      const uint32_t h1 = hdr[1];
      n = h1 ? h1 : 256u;
      hb = 2;
      if (n < 128) err = 1;
    }
  } else {
    n = h0 & 0x7Fu;
    hb = 1;
    if (n == 0) err = 1;
  }
  if (!err && hdr_avail < hb + (n + 1) / 2) err = 1;
  uint32_t w = 0;
  if (!err && t < n) {
    const uint32_t b = hdr[hb + t / 2];
    w = (t % 2 == 0) ? (b & 0x0Fu) : ((b >> 4) & 0x0Fu);
  }
  // per wavefront: symbols of each length and rank among them; [0]: any
  // length above 11
  const bool too_long = w > 11;
  if (too_long) w = 0;
  uint32_t rank = 0;
#pragma unroll
  for (uint32_t l = 1; l <= 11; ++l) {
    const uint64_t m = __ballot(w == l);
    if (w == l) rank = __popcll(m & ((1ull << lane) - 1ull));
    if (lane == 0) bs.wave_len_count[wave][l] = __popcll(m);
  }
  const uint64_t tl = __ballot(too_long);
  if (lane == 0) bs.wave_len_count[wave][0] = tl ? 1u : 0u;
  __syncthreads();
  // symbols per length (threads 1..11), then the canonical codes, offsets
  // and limits (thread 0, eleven steps)
  if (t >= 1 && t <= 11)
    bs.cnt[t] = bs.wave_len_count[0][t] + bs.wave_len_count[1][t] + bs.wave_len_count[2][t] + bs.wave_len_count[3][t];
  uint32_t before = 0;
  for (uint32_t wv = 0; wv < wave; ++wv) before += w ? bs.wave_len_count[wv][w] : 0u;
  __syncthreads();
  if (t == 0) {
    if (bs.wave_len_count[0][0] | bs.wave_len_count[1][0] | bs.wave_len_count[2][0] | bs.wave_len_count[3][0]) err = 1;
    uint32_t code = 0, off = 0, kraft = 0, total = 0, max_bits = 0, cprev = 0;
    for (uint32_t l = 1; l <= 11; ++l) {
      const uint32_t c = bs.cnt[l];
      code = (code + cprev) << 1;  // first code of length l
      if (c && code + c > (1u << l)) err = 1;
      bs.off[l] = off;
      bs.base[l] = off - code;
      bs.lim[l] = (code + c) << (11 - l);
      off += c;
      total += c;
      kraft += c << (11 - l);
      if (c) max_bits = l;
      cprev = c;
    }
    if (total == 0 || kraft > 2048) err = 1;
    if (max_bits < 1) max_bits = 1;
    bs.err = err;
    bs.max_bits = max_bits;
    bs.hdr_len = hb + (n + 1) / 2;
    bs.pair = pair_ok && n <= 16 && max_bits <= 6 ? 1u : 0u;
  }
  __syncthreads();
  err = bs.err;
  const uint32_t max_bits = bs.max_bits;
  const bool pair = bs.pair;
  if (w && !err) bs.sorted[bs.off[w] + before + rank] = (uint8_t)t;  // symbols in canonical order
  // the limits, uniform: scalar registers
  uint32_t lim[12];
#pragma unroll
  for (uint32_t l = 1; l <= 11; ++l) lim[l] = __builtin_amdgcn_readfirstlane(bs.lim[l]);
  __syncthreads();
  if (pair) {
    // 6-bit single tables (raw symbols and symbol'), then the pair table:
    // the two codes at the start of each 12-bit window (both <= 6 bits)
    if (t < 64) {
      const uint32_t v = (__builtin_bitreverse32(t) >> 26) << 5;
      uint32_t len = 1;
#pragma unroll
      for (uint32_t l = 1; l <= 10; ++l) len += v >= lim[l] ? 1u : 0u;
      uint32_t e = max_bits, er = max_bits;
      if (v < lim[11] && !err) {
        const uint32_t sym = bs.sorted[bs.base[len] + (v >> (11 - len))];
        e = len | (xform_byte(xf, sym) << 8);
        er = len | (sym << 8);
      }
      t64[t] = (uint16_t)e;
      bs.t64raw[t] = (uint16_t)er;
    }
    __syncthreads();
    const uint32_t e0 = bs.t64raw[t & 63u];  // window bits 0..5 of every i = t + 256 k
    const uint32_t l0 = e0 & 0xFFu;
#pragma unroll 4
    for (uint32_t k = 0; k < 16; ++k) {
      const uint32_t i = t + 256 * k;
      const uint32_t e1 = bs.t64raw[(i >> l0) & 63u];
      tab[i] = (uint16_t)((l0 + (e1 & 0xFFu)) | ((e0 >> 8) << 8) | ((e1 >> 8) << 12));
    }
    __syncthreads();
    return;
  }
  // single table: a window matching no code (incomplete code) decodes as
  // symbol 0 (every transform maps 0 to 0) with length max_bits
#pragma unroll 1
  for (uint32_t k = 0; k < 8; ++k) {
    const uint32_t i = t + 256 * k;
    const uint32_t v = __builtin_bitreverse32(i) >> 21;
    uint32_t len = 1;
#pragma unroll
    for (uint32_t l = 1; l <= 10; ++l) len += v >= lim[l] ? 1u : 0u;
    uint32_t e = max_bits;
    if (v < lim[11] && !err) e = len | (xform_byte(xf, bs.sorted[bs.base[len] + (v >> (11 - len))]) << 8);
    tab[i] = (uint16_t)e;
  }
  __syncthreads();
}

// q + (e & 0xFF) in one instruction (SDWA byte select of the VOP2 add).
__device__ __forceinline__ uint32_t add_byte0(uint32_t q, uint32_t e) {
  uint32_t r;
  asm("v_add_u32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0 src1_sel:DWORD"
      : "=v"(r)
      : "v"(e), "v"(q));
  return r;
}

// Entry-address masks: window bits 1..11 (single table), 1..12 (pair
// table), 1..6 (the 64-entry tables), each times the 2-byte entry size.
constexpr uint32_t kMask11 = 0xFFEu, kMask12 = 0x1FFEu, kMask6 = 0x7Eu;

// LDS address of the table entry for a window: (win & kMask) | lut (lut is a
// multiple of the table size).  One v_and_or_b32 with the mask in a VGPR:
// gfx9 VOP3 has no literal operand and reads at most one SGPR.
template <uint32_t kMask>
__device__ __forceinline__ uint32_t lut_entry_addr(uint32_t win, uint32_t lut) {
  if (__builtin_constant_p(lut) && lut == 0) return win & kMask;
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(win), "v"(kMask), "s"(lut));
  return r;
}

// Pack the symbol bytes (byte 1 of each entry) of 16 entries into 4 words.
__device__ __forceinline__ void pack_symbols(const uint32_t (&e)[16], uint32_t (&v)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t a = __builtin_amdgcn_perm(e[4 * j + 1], e[4 * j], 0x0c0c0501u);
    const uint32_t b = __builtin_amdgcn_perm(e[4 * j + 3], e[4 * j + 2], 0x05010c0cu);
    v[j] = a | b;
  }
}

// Decode one group (16 symbols; with kTail only the first `count` advance
// the stream) from the wavefront's staged words.  qm = the lane's absolute
// LDS bit address minus one: bit 0 of each window is the bit before the next
// code, so `window & kMask` is directly the byte offset of its entry in the
// single-mode table at LDS address `lut`.  Reads stay inside the
// workgroup's staging area: a lane reads at most 90 words past its first
// word, and the area ends with 96 spare words.
template <bool kTail, uint32_t kMask>
__device__ __forceinline__ void group_lds(uint32_t lut, uint32_t& qm, uint32_t count, uint32_t (&v)[4]) {
  uint32_t e[16];
#pragma unroll
  for (uint32_t k = 0; k < 16; k += 2) {
    const uint32_t wa = (qm >> 3) & ~3u;
    const uint32_t win = __builtin_amdgcn_alignbit(lds_ld32(wa + 4), lds_ld32(wa), qm);
    const uint32_t e0 = lds_ld16(lut_entry_addr<kMask>(win, lut));
    // the shift uses the low 5 bits of the entry: its code length
    const uint32_t win1 = __builtin_amdgcn_alignbit(0u, win, kTail && k >= count ? 0u : e0);
    const uint32_t e1 = lds_ld16(lut_entry_addr<kMask>(win1, lut));
    if constexpr (kTail) {
      const uint32_t l0 = k >= count ? 0u : (e0 & 0xFFu);
      const uint32_t l1 = k + 1 >= count ? 0u : (e1 & 0xFFu);
      qm += l0 + l1;
    } else {
      qm = add_byte0(add_byte0(qm, e0), e1);
    }
    e[k] = e0;
    e[k + 1] = e1;
  }
  pack_symbols(e, v);
}

// A lane's staged stream with its next words held in registers (the fast
// path's reader).  The window of two lookups comes from w0:w1 with one
// alignbit, so the dependent chain of a step is the two table lookups; the
// word after w1 is read from LDS at the end of every step (a re-read of the
// same word when no word was finished), one step before it can be needed.
// A step consumes at most 22 bits, so bo stays below 32 + 22 and at most
// one word is finished per step.
struct BitReg {
  uint32_t w0, w1, w2;  // stream words j, j + 1, j + 2 (word -1 reads as 0)
  uint32_t bo;          // bit of w0 just before the next code
  uint32_t wp;          // LDS byte address of word j + 2
};

// From the reader position qm (LDS bit address of the lane's first word,
// minus one: the state before the lane's first code).
__device__ __forceinline__ BitReg bitreg_open(uint32_t qm) {
  const uint32_t wa = (qm + 1u) >> 3;
  return BitReg{0u, lds_ld32(wa), lds_ld32(wa + 4), 31u, wa + 4};
}

// The reader position qm0 + bits consumed (32 j + bo + 1), for the
// acceptance check.
__device__ __forceinline__ uint32_t bitreg_close(const BitReg& b, uint32_t qm0) {
  const uint32_t wa = (qm0 + 1u) >> 3;
  return qm0 + 8u * (b.wp - wa) - 63u + b.bo;
}

__device__ __forceinline__ uint32_t bitreg_window(const BitReg& b) {
  return __builtin_amdgcn_alignbit(b.w1, b.w0, b.bo);
}

// bo_next = bo + the step's code bits (< 64)
__device__ __forceinline__ void bitreg_step(BitReg& b, uint32_t bo_next) {
  const bool s = bo_next >= 32u;
  b.w0 = s ? b.w1 : b.w0;
  b.w1 = s ? b.w2 : b.w1;
  b.wp += s ? 4u : 0u;
  b.bo = bo_next & 31u;
  b.w2 = lds_ld32(b.wp);
}

// group_lds<false, kMask> from the register reader
template <uint32_t kMask>
__device__ __forceinline__ void group_reg(uint32_t lut, BitReg& b, uint32_t (&v)[4]) {
  uint32_t e[16];
#pragma unroll
  for (uint32_t k = 0; k < 16; k += 2) {
    const uint32_t win = bitreg_window(b);
    const uint32_t e0 = lds_ld16(lut_entry_addr<kMask>(win, lut));
    const uint32_t e1 = lds_ld16(lut_entry_addr<kMask>(__builtin_amdgcn_alignbit(0u, win, e0), lut));
    bitreg_step(b, add_byte0(add_byte0(b.bo, e0), e1));
    e[k] = e0;
    e[k + 1] = e1;
  }
  pack_symbols(e, v);
}

// Pair mode, full group: 8 lookups in the 12-bit pair table at `lut`, one
// 32-bit window per two lookups (<= 24 code bits plus the leading bit).
// Yields the 16 raw nibble symbols, one per byte.
__device__ __forceinline__ void group_lds_pair(uint32_t lut, uint32_t& qm, uint32_t (&v)[4]) {
#pragma unroll
  for (uint32_t j = 0; j < 4; ++j) {
    const uint32_t wa = (qm >> 3) & ~3u;
    const uint32_t win = __builtin_amdgcn_alignbit(lds_ld32(wa + 4), lds_ld32(wa), qm);
    const uint32_t e0 = lds_ld16(lut_entry_addr<kMask12>(win, lut));
    const uint32_t e1 = lds_ld16(lut_entry_addr<kMask12>(__builtin_amdgcn_alignbit(0u, win, e0), lut));
    qm = add_byte0(add_byte0(qm, e0), e1);
    // [s0|s1<<4, 0, s2|s3<<4, 0] -> one nibble per byte
    const uint32_t w = __builtin_amdgcn_perm(e1, e0, 0x0c050c01u);
    v[j] = (w | (w << 4)) & 0x0F0F0F0Fu;
  }
}

// Two pair-mode planes of one block (plane a at table la, plane b at lb):
// the same steps as group_lds_pair, with the two independent lookup chains
// interleaved so that each one's LDS latency overlaps the other's work.
__device__ __forceinline__ void group_lds_pair2(uint32_t la, uint32_t& qa, uint32_t (&va)[4], uint32_t lb,
                                                uint32_t& qb, uint32_t (&vb)[4]) {
#pragma unroll
  for (uint32_t j = 0; j < 4; ++j) {
    const uint32_t wa = (qa >> 3) & ~3u, wb = (qb >> 3) & ~3u;
    const uint32_t xa = __builtin_amdgcn_alignbit(lds_ld32(wa + 4), lds_ld32(wa), qa);
    const uint32_t xb = __builtin_amdgcn_alignbit(lds_ld32(wb + 4), lds_ld32(wb), qb);
    const uint32_t a0 = lds_ld16(lut_entry_addr<kMask12>(xa, la));
    const uint32_t b0 = lds_ld16(lut_entry_addr<kMask12>(xb, lb));
    const uint32_t a1 = lds_ld16(lut_entry_addr<kMask12>(__builtin_amdgcn_alignbit(0u, xa, a0), la));
    const uint32_t b1 = lds_ld16(lut_entry_addr<kMask12>(__builtin_amdgcn_alignbit(0u, xb, b0), lb));
    qa = add_byte0(add_byte0(qa, a0), a1);
    qb = add_byte0(add_byte0(qb, b0), b1);
    const uint32_t ua = __builtin_amdgcn_perm(a1, a0, 0x0c050c01u);
    const uint32_t ub = __builtin_amdgcn_perm(b1, b0, 0x0c050c01u);
    va[j] = (ua | (ua << 4)) & 0x0F0F0F0Fu;
    vb[j] = (ub | (ub << 4)) & 0x0F0F0F0Fu;
  }
}

// Fallback for a block that does not fit the staging budget: the same
// decode reading the lane's words (nw of them) from global memory; words
// past the lane's count read as zero, as in the specification decoder.
// q = bits consumed by the lane so far.  kMask selects the single-mode
// table (11-bit) or a pair-mode plane's 64-entry table.
template <uint32_t kMask>
__device__ __forceinline__ void group_global(uint32_t lut, const uint32_t* words, uint32_t nw, uint32_t& q,
                                             uint32_t count, uint32_t (&v)[4]) {
  uint32_t e[16];
#pragma unroll
  for (uint32_t k = 0; k < 16; k += 2) {
    const uint32_t wi = q >> 5;
    const uint32_t lo = wi < nw ? gload_u32(words + wi) : 0u;
    const uint32_t hi = wi + 1 < nw ? gload_u32(words + wi + 1) : 0u;
    const uint32_t win = __builtin_amdgcn_alignbit(hi, lo, q);
    const uint32_t e0 = lds_ld16(lut + ((win << 1) & kMask));
    const uint32_t l0 = k < count ? (e0 & 0xFFu) : 0u;
    const uint32_t e1 = lds_ld16(lut + ((__builtin_amdgcn_alignbit(0u, win, l0) << 1) & kMask));
    const uint32_t l1 = k + 1 < count ? (e1 & 0xFFu) : 0u;
    q += l0 + l1;
    e[k] = e0;
    e[k + 1] = e1;
  }
  pack_symbols(e, v);
}

static_assert(sizeof(DecodeCtl) <= 3072, "LDS control block stays small");

}  // namespace

// ---------------------------------------------------------------------------
// decode (fused with the inverse chain)
// ---------------------------------------------------------------------------

// LDS table slot size of a chain's coded planes (pair-mode capable or not).
__host__ __device__ constexpr uint32_t chain_slot_bytes(uint32_t chain) {
  // a two-chain launch: the larger of its chains' slots
  return ilv_is_pair(chain) ? (chain_slot_bytes(ilv_pair_a(chain)) > chain_slot_bytes(ilv_pair_b(chain))
                                   ? chain_slot_bytes(ilv_pair_a(chain))
                                   : chain_slot_bytes(ilv_pair_b(chain)))
         : chain == kChainIeee16Split2 || chain == kChainIeee32Split4 ? kIlvLutBytes
                                                                        : kIlvPairLutBytes;
}

template <uint32_t C>
struct ChainTag {
  static constexpr uint32_t value = C;
};

// Per-block state of one wavefront: for each plane, a raw-byte base or a
// coded stream (staged: absolute LDS bit address; global: lane word pointer,
// word count and bits consumed).
template <uint32_t NP>
struct BlockState {
  uint64_t raw[NP];
  const uint32_t* words[NP];
  uint32_t nw[NP];
  uint32_t q[NP];
  uint32_t t64[NP];     // LDS address of a pair-mode plane's 64-entry table
  uint32_t lut[NP];     // LDS address of a coded plane's table
  uint32_t rbytes[NP];   // bytes of a raw plane's data (0 for a coded plane)
  uint32_t coded_mask;   // bit p: plane p is huff_ilv coded
  uint32_t pair_mask;    // bit p: plane p decodes in pair mode
  uint32_t packed_mask;  // bit p: plane p is stored as packed nibbles
};

// Load the raw (uncoded) planes' bytes of the group at plane position pos:
// full blocks with aligned planes issue one load per plane (expanded by the
// consumer), other blocks load and expand the group's symbols.
// kSkipCoded (plane forms fixed at compile time): coded planes issue no load.
template <uint32_t kChain, bool kTail, bool kSkipCoded = false>
__device__ __forceinline__ void load_raw(const BlockState<ChainInfo<kChain>::np>& st, uint32_t coded_mask,
                                         uint32_t packed_mask, uint64_t pos, uint64_t n,
                                         uint32_t (&x)[ChainInfo<kChain>::np][4], bool live = true) {
  constexpr uint32_t NP = ChainInfo<kChain>::np;
#pragma unroll
  for (uint32_t p = 0; p < NP; ++p) {
    if constexpr (kTail) {
      if (coded_mask & (1u << p)) continue;
      load_group(st.raw[p], (packed_mask >> p) & 1u, pos, group_count<kTail>(pos, n), x[p]);
    } else {
      if (kSkipCoded && (coded_mask & (1u << p))) continue;
      load_group_fast(st.raw[p], st.rbytes[p], (packed_mask >> p) & 1u, (uint32_t)pos, live, x[p]);
    }
  }
}

// The 16 rounds of one block: decode one group per coded plane, take the
// raw planes' groups (loaded one round ahead, so their latency overlaps the
// table lookups), merge and store.  luts: LDS address of the first table
// slot; plane p uses the table at st.lut[p].  out: output tensor address.
//
// kCrc (crc_on uniform, whole blocks only): acc[p] becomes the zero-init
// CRC-32 of the lane's 16 pieces of plane p (pieces 1 KiB apart), relative
// to the end of its last piece: acc' = acc x^(8 * 1024) xor crc0(piece).
// crc0 by slicing-by-4 (Kounavis & Berry) and the advance by four
// byte-sliced lookups, from tables at LDS address 0 (crc_round_lds0); a
// plane whose symbols are held rotated is rotated back first.
template <uint32_t kChain, bool kTail, bool kStaged, bool kCrc = false, uint32_t kFix = 0>
__device__ __forceinline__ void decode_block(BlockState<ChainInfo<kChain>::np>& st, uint32_t luts, uint64_t out,
                                             uint64_t n, uint64_t bstart, uint32_t lane,
                                             uint32_t* acc = nullptr) {
  constexpr uint32_t NP = ChainInfo<kChain>::np;
  constexpr uint32_t RATIO = ChainInfo<kChain>::ratio;
  static_assert(kFix == 0 || (!kTail && kStaged), "fixed plane forms: fast staged path only");
  const uint32_t coded_mask = kFix ? kFix - 1 : st.coded_mask;
  const uint32_t pair_mask = kFix ? 0u : st.pair_mask;
  const uint32_t packed_mask = kFix ? 0u : st.packed_mask;
  static_assert(kIlvCrcWords == kCrcLdsWords, "LDS copy of the CRC tables");
  // the fixed-form fast path reads the coded planes' staged streams through
  // registers (elsewhere the readers' extra registers cost more occupancy
  // than the shorter lookup chain gains)
  constexpr bool kReg = kStaged && !kTail && kFix != 0;
  BitReg br[NP];
  if constexpr (kReg) {
#pragma unroll
    for (uint32_t p = 0; p < NP; ++p)
      if (coded_mask & (1u << p)) br[p] = bitreg_open(st.q[p]);
  }
  uint32_t nxt[NP][4];
  load_raw<kChain, kTail, kFix != 0>(st, coded_mask, packed_mask, bstart + (uint64_t)kIlvGroup * lane, n, nxt);
  if constexpr (!kTail) {
#pragma unroll
    for (uint32_t k = 0; k < RATIO; ++k) vmem_nop(out, k);
  }
  for (uint32_t r = 0; r < kIlvRounds; ++r) {
    const uint64_t pos = bstart + (uint64_t)kIlvGroup * (r * 64u + lane);
    const uint32_t count = group_count<kTail>(pos, n);
    uint32_t v[NP][4];
    bool done = false;
    if constexpr (NP == 2 && kStaged && !kTail) {
      if (coded_mask == 3u && pair_mask == 3u) {
        // both nibble planes in pair mode: their two lookup chains interleaved
        group_lds_pair2(st.lut[0], st.q[0], v[0], st.lut[1], st.q[1], v[1]);
#pragma unroll
        for (uint32_t p = 0; p < 2; ++p)
#pragma unroll
          for (int k = 0; k < 4; ++k) v[p][k] = xform_word(ChainInfo<kChain>::xf[p], v[p][k]);
        done = true;
      }
    }
#pragma unroll
    for (uint32_t p = 0; p < NP; ++p) {
      if (done || !(coded_mask & (1u << p))) continue;
      const uint32_t lut = st.lut[p];
      if (pair_mask & (1u << p)) {
        if constexpr (kStaged && !kTail) {
          group_lds_pair(lut, st.q[p], v[p]);
#pragma unroll
          for (int k = 0; k < 4; ++k) v[p][k] = xform_word(ChainInfo<kChain>::xf[p], v[p][k]);
        } else if constexpr (kStaged) {
          group_lds<kTail, kMask6>(st.t64[p], st.q[p], count, v[p]);
        } else {
          group_global<kMask6>(st.t64[p], st.words[p], st.nw[p], st.q[p], count, v[p]);
        }
      } else {
        if constexpr (kReg) group_reg<kMask11>(lut, br[p], v[p]);
        else if constexpr (kStaged) group_lds<kTail, kMask11>(lut, st.q[p], count, v[p]);
        else group_global<kMask11>(lut, st.words[p], st.nw[p], st.q[p], count, v[p]);
      }
    }
#pragma unroll
    for (uint32_t p = 0; p < NP; ++p) {
      if constexpr (kTail) {
        if (coded_mask & (1u << p)) continue;
#pragma unroll
        for (int k = 0; k < 4; ++k) v[p][k] = xform_word(ChainInfo<kChain>::xf[p], nxt[p][k]);
      } else {
        // every plane's load is consumed here (coded planes loaded zeros,
        // or nothing with fixed plane forms)
        const bool raw = !(coded_mask & (1u << p));
        if (kFix && !raw) continue;
        uint32_t x[4];
        expand_group((packed_mask >> p) & 1u, nxt[p], x);
#pragma unroll
        for (int k = 0; k < 4; ++k) v[p][k] = raw ? xform_word(ChainInfo<kChain>::xf[p], x[k]) : v[p][k];
      }
    }
    if constexpr (kTail) {
      if (r + 1 < kIlvRounds) load_raw<kChain, kTail, kFix != 0>(st, coded_mask, packed_mask, pos + (uint64_t)kIlvGroup * 64u, n, nxt);
    } else {
      load_raw<kChain, kTail, kFix != 0>(st, coded_mask, packed_mask, pos + (uint64_t)kIlvGroup * 64u, n, nxt, r + 1 < kIlvRounds);
    }
    if constexpr (kCrc) {
#pragma unroll
      for (uint32_t p = 0; p < NP; ++p) {
        const uint32_t xf = ChainInfo<kChain>::xf[p];
        acc[p] = crc_round_lds0(acc[p], u32x4_make(unxform_word(xf, v[p][0]), unxform_word(xf, v[p][1]),
                                                   unxform_word(xf, v[p][2]), unxform_word(xf, v[p][3])));
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
  if constexpr (kReg) {
#pragma unroll
    for (uint32_t p = 0; p < NP; ++p)
      if (coded_mask & (1u << p)) st.q[p] = bitreg_close(br[p], st.q[p]);
  }
}

// tensors: all tensors of the call; tix[j]: the tensor of this launch's j-th
// entry, whose 4-block tiles are tpre[j] .. tpre[j+1] - 1 (m entries,
// n_tiles = tpre[m]).  Workgroup g takes tiles [g n_tiles / G, (g+1) n_tiles / G).
// Four wavefronts per SIMD (four workgroups per CU, the LDS budget of the
// one- and two-coded-plane chains) need at most 128 VGPRs per lane; the
// four-plane IEEE-32 chain runs at two workgroups per CU (256 VGPRs).  The
// fused-CRC variants get no cap: held to 128 VGPRs they spill, and their
// headline launch ran 7.98 ms against 7.2 ms uncapped.
template <uint32_t kChain, bool kCrc>
__global__ void __launch_bounds__(256)
    __attribute__((amdgpu_waves_per_eu(kCrc ? 1 : kChain == kChainIeee32Split4 ? 2 : 4)))
ilv_decode_kernel(IlvInline inl_arg, const IlvTensor* __restrict__ tensors, const uint32_t* __restrict__ tix_mem,
                  const uint32_t* __restrict__ tpre_mem, uint32_t m_mem, uint32_t* __restrict__ status,
                  uint32_t n_slots, uint32_t stage_words, const uint32_t* __restrict__ crc_tab,
                  uint32_t* __restrict__ crc_part) {
  // Descriptors from the kernel arguments or from device memory, both read
  // through constant-address-space pointers (uniform: scalar loads).  The
  // inline ones are read in place (the first argument: offset 0 of the
  // kernel argument segment); naming the by-value argument would copy it to
  // per-lane scratch.
  (void)inl_arg;
  const KConst IlvInline& inl = *(const KConst IlvInline*)__builtin_amdgcn_kernarg_segment_ptr();
  const bool inl_on = inl.m != 0;
  const uint32_t m = inl_on ? inl.m : m_mem;
  const KConst uint32_t* const tix = inl_on ? inl.tix : (const KConst uint32_t*)tix_mem;
  const KConst uint32_t* const tpre = inl_on ? inl.tpre : (const KConst uint32_t*)tpre_mem;
  constexpr uint32_t SLOT = chain_slot_bytes(kChain);
  // The kernel has no static LDS, so the dynamic area starts at LDS address
  // 0 and every table sits on a SLOT boundary (entry address =
  // (window & mask) | table base).  Layout:
  //   [kCrc: CRC tables, 8 KiB at address 0 (crc_round_lds0)]
  //   [n_slots tables (coded planes from the last one down)][DecodeCtl]
  //   [4 wavefronts x stage_words][96 spare words]
  extern __shared__ __align__(16) uint8_t lds[];
  uint8_t* const smem = lds + (kCrc ? 4u * kIlvCrcWords : 0u);
  DecodeCtl& ctl = *reinterpret_cast<DecodeCtl*>(smem + n_slots * SLOT);
  uint32_t* const stage = reinterpret_cast<uint32_t*>(smem + n_slots * SLOT + sizeof(DecodeCtl));
  // while a tensor's tables are built, the staging area holds the payload
  // heads (the host sizes it for NP x kIlvHeadWords words at least)
  uint32_t (*const head)[kIlvHeadWords] = reinterpret_cast<uint32_t (*)[kIlvHeadWords]>(stage);
  const uint32_t luts = lds_addr(smem);
  BuildScratch& bs = ctl.bs;
  uint64_t* const s_table = ctl.table;
  uint64_t* const s_data = ctl.data;
  uint64_t* const s_datalen = ctl.datalen;
  uint64_t* const s_raw = ctl.raw;
  uint32_t* const s_coded = ctl.coded;
  uint32_t* const s_pair = ctl.pair;
  uint32_t& s_bad = ctl.bad;
  const uint32_t t = threadIdx.x, wave = t >> 6, lane = t & 63u;
  if (luts & (SLOT - 1)) {
    // not reachable with the layout above; refuse rather than mis-decode
    if (t == 0 && blockIdx.x == 0) status_or(&status[tix[0]], kIlvErrHeader);
    return;
  }
  const uint32_t n_tiles = tpre[m];
  const uint32_t tile0 = (uint32_t)((uint64_t)blockIdx.x * n_tiles / gridDim.x);
  const uint32_t tile1 = (uint32_t)((uint64_t)(blockIdx.x + 1) * n_tiles / gridDim.x);
  if (tile0 >= tile1) return;
  // entry holding tile0: the last j with tpre[j] <= tile0
  uint32_t lo = 0, hi = m;
  while (hi - lo > 1) {
    const uint32_t mid = (lo + hi) / 2;
    if (tpre[mid] <= tile0) lo = mid;
    else hi = mid;
  }
  uint32_t j = lo, cur = 0xFFFFFFFFu, bad = 0;
  uint32_t* const sw = stage + wave * stage_words;
  // CRC nibble tables N, NR, NA (visible after the first tile's barriers)
  if constexpr (kCrc) {
    // T0..T3 and the byte-sliced advance over 1 KiB
    uint32_t* const crcT = reinterpret_cast<uint32_t*>(lds);
    if (lds_addr(crcT) != 0) {  // not reachable: the kernel has no static LDS
      if (t == 0 && blockIdx.x == 0) status_or(&status[tix[0]], kIlvErrHeader);
      return;
    }
    for (uint32_t i = t; i < kIlvCrcWords; i += 256) crcT[i] = crc_tab[i < 1024 ? i : i - 1024 + kCrcTabS1024];
  }
  // At a tensor's first tile each wavefront requests its block's offsets
  // as soon as the payload heads are in LDS (while thread 0 parses them),
  // then its lane counts, and touches every 128-byte line of the block
  // before the tables are built (loads into one discarded register), so that
  // the copy into LDS after the build reads from the L2 cache: the parse and
  // the build hide the memory latency.
  for (uint32_t tile = tile0; tile < tile1; ++tile) {
    while (tile >= tpre[j + 1]) ++j;
    const uint32_t ti = tix[j];
    const KConst IlvTensor& T = inl_on ? inl.t[j] : *(const KConst IlvTensor*)(tensors + ti);
    // the tile, decoded by the code of its tensor's chain (a two-chain
    // launch holds both)
    auto body = [&](auto tag) {
      constexpr uint32_t C = decltype(tag)::value;
      constexpr uint32_t NP = ChainInfo<C>::np;
      const uint64_t n = T.n;
      const uint32_t nb = (uint32_t)((n + kIlvBlock - 1) / kIlvBlock);
      const uint32_t bi = kIlvBlocksPerTile * (tile - tpre[j]) + wave;
      // ---- block geometry of the wavefront's block (one wavefront per block) ----
      BlockState<NP> st;
      uint32_t lane_c[NP], tot[NP], first[NP];
      uint32_t need = 4, need_skew = 0, uni_mask = 0;
      bool ok = true, prepped = false, early = false;
      uint32_t e_o0[NP], e_o1[NP], e_c[NP];  // offsets and count read before the build
      uint32_t e_ready = 0;                  // planes whose e_o0 / e_o1 are requested
      // block [o0, o1) of coded plane p; c = lane's word count (0 if rejected)
      // offsets of an accepted stream are multiples of 4 (tab[0] == 0 and
      // every block is 64 + 4 x words bytes long)
      auto block_ok = [&](uint32_t p, uint32_t o0, uint32_t o1) -> bool {
        return o1 >= o0 && o1 <= s_datalen[p] && o1 - o0 >= 64 && (o0 & 3u) == 0 && (bi != 0 || o0 == 0) &&
               (bi + 1 != nb || o1 == s_datalen[p]);
      };
      auto block_head = [&](uint32_t p, uint32_t& o0, uint32_t& o1, uint32_t& c) -> bool {
        const uint32_t* tab = reinterpret_cast<const uint32_t*>(s_table[p]);
        o0 = gload_u32(tab + bi);
        o1 = gload_u32(tab + bi + 1);
        const bool bok = block_ok(p, o0, o1);
        c = bok ? gload_u8(s_data[p] + o0 + lane) : 0u;
        return bok;
      };
      // Loads issued here are consumed only after the build; every load is
      // unconditional, with `safe` (the tensor descriptor) as the address of
      // one that is not wanted, so no result is moved before it arrives.
      const uint64_t safe = reinterpret_cast<uint64_t>(&T.n);
      uint32_t e_touch[NP][2];
      auto touch = [&]() {
        early = true;
#pragma unroll
        for (uint32_t p = 0; p < NP; ++p) {
          uint32_t o0 = 0, o1 = 0;
          bool bok = false;
          if (__builtin_amdgcn_readfirstlane(s_coded[p])) {
            if ((e_ready >> p) & 1u) {
              o0 = e_o0[p];
              o1 = e_o1[p];
              bok = block_ok(p, o0, o1);
            } else {
              uint32_t c;
              bok = block_head(p, o0, o1, c);
            }
          }
          // a rejected block reads as empty (prep then rejects it)
          e_o0[p] = bok ? o0 : 0u;
          e_o1[p] = bok ? o1 : 0u;
          // the lane count, and the block's 128-byte lines (all inside the
          // plane's data); blocks are at most 16 KiB + 64 bytes in practice,
          // longer ones are read from memory after the build.  (Touching the
          // raw planes' blocks as well was slower: the decode that reads them
          // is bound by its VALU work, and the touches delay the staging.)
          const uint64_t b = s_data[p] + o0;
          const uint32_t len = bok ? o1 - o0 : 0u;
          // (the word holding the lane's count byte: o0 is a multiple of 4)
          e_c[p] = g_ld<uint32_t>(bok ? b + (lane & ~3u) : safe);
          e_touch[p][0] = g_ld<uint32_t>(128 * lane < len ? b + 128 * lane : safe);
          e_touch[p][1] = g_ld<uint32_t>(8192 + 128 * lane < len ? b + 8192 + 128 * lane : safe);
        }
      };
      auto prep = [&]() {
        prepped = true;
        st.coded_mask = 0;
        st.pair_mask = 0;
        st.packed_mask = 0;
#pragma unroll
        for (uint32_t p = 0; p < NP; ++p) {
          st.raw[p] = s_raw[p];
          if (__builtin_amdgcn_readfirstlane(ctl.packed[p])) st.packed_mask |= 1u << p;
          st.words[p] = nullptr;
          st.nw[p] = 0;
          st.q[p] = 0;
          st.t64[p] = lds_addr(ctl.t64[p]);
          st.lut[p] = luts + __builtin_amdgcn_readfirstlane(ctl.slot[p]) * SLOT;
          lane_c[p] = tot[p] = first[p] = 0;
          if (!__builtin_amdgcn_readfirstlane(s_coded[p])) continue;
          st.coded_mask |= 1u << p;
          uint32_t o0, o1, c;
          bool bok;
          if (early) {
            o0 = e_o0[p];
            o1 = e_o1[p];
            bok = o1 - o0 >= 64;  // touch() leaves both 0 for a rejected block
            c = bok ? (e_c[p] >> (8 * (lane & 3u))) & 0xFFu : 0u;
          } else {
            bok = block_head(p, o0, o1, c);
          }
          const uint8_t* blk = reinterpret_cast<const uint8_t*>(s_data[p]) + (bok ? o0 : 0);
          const uint32_t incl = wave_incl_scan(c);
          const uint32_t total = __shfl(incl, 63, 64);
          if (!bok || 64u + 4u * total != o1 - o0) ok = false;
          st.words[p] = reinterpret_cast<const uint32_t*>(blk + 64);
          lane_c[p] = c;
          tot[p] = total;
          first[p] = incl - c;
          need += (total + 3u) & ~3u;
          const uint32_t c0 = __builtin_amdgcn_readfirstlane(c);
          if (__ballot(c != c0) == 0 && c0 >= 4) {
            uni_mask |= 1u << p;
            need_skew += 128u;  // room for up to two skew words per lane
          }
        }
      };
      if (ti != cur) {
        // ---- new tensor: parse its plane headers and build the LDS tables ----
        bad = wave_or_status(bad);
        if (bad && lane == 0) status_or(&status[cur], bad);
        bad = 0;
        cur = ti;
        __syncthreads();  // every wavefront is done with the previous tables
        // the payload heads (tag, n, weights header) and last bytes, loaded
        // by all threads at once (coded payloads start 4-byte aligned)
        for (uint32_t k = t; k < NP * (kIlvHeadWords + 1); k += 256) {
          const uint32_t p = k / (kIlvHeadWords + 1), w = k % (kIlvHeadWords + 1);
          const uint64_t base = T.planes[p].base, len = T.planes[p].len;
          uint32_t v = 0;
          if (T.planes[p].coded) {
            if (w == kIlvHeadWords) {
              if (len) v = gload_u8(base + len - 1);
            } else if (4ull * w + 4 <= len) {
              v = g_ld<uint32_t>(base + 4ull * w);
            } else {
              for (uint64_t b = 4ull * w; b < len && b < 4ull * w + 4; ++b) v |= gload_u8(base + b) << (8 * (b & 3));
            }
          }
          if (w == kIlvHeadWords) ctl.last[p] = v;
          else head[p][w] = v;
        }
        if (t < NP) {
          ctl.pbase[t] = T.planes[t].base;
          ctl.plen[t] = T.planes[t].len;
          ctl.pcoded[t] = T.planes[t].coded;
        }
        __syncthreads();
        // the block's offsets, requested while thread 0 parses the heads
#pragma unroll
        for (uint32_t p = 0; p < NP; ++p) {
          const uint64_t len = ctl.plen[p];
          const uint8_t* pay = reinterpret_cast<const uint8_t*>(head[p]);
          uint64_t tb = 0, dt = 0;
          const bool v = bi < nb && ctl.pcoded[p] && len >= 5 && pay[0] == 1 &&
                         coded_layout(pay, (uint32_t)(len < 4 * kIlvHeadWords ? len : 4 * kIlvHeadWords), len, nb, tb, dt);
          // tb + 4 (bi + 2) <= dt <= len: inside the payload
          const uint64_t a = ctl.pbase[p] + tb + 4ull * bi;
          e_o0[p] = g_ld<uint32_t>(v ? a : safe);
          e_o1[p] = g_ld<uint32_t>(v ? a + 4 : safe);
          if (v) e_ready |= 1u << p;
        }
        if (t == 0) {
          s_bad = 0;
          for (uint32_t p = 0; p < NP; ++p) {
            const uint64_t base = ctl.pbase[p], len = ctl.plen[p];
            s_raw[p] = base;
            s_coded[p] = 0;
            ctl.packed[p] = 0;
            if (!ctl.pcoded[p]) continue;
            // huff_ilv payload: tag 0 stores the plane after the tag byte, tag 2 packs it
            const uint8_t* pay = reinterpret_cast<const uint8_t*>(head[p]);
            if (len == 0) s_bad |= kIlvErrHeader;
            else if (pay[0] == 0) {
              if (len != n + 1) s_bad |= kIlvErrHeader;
              s_raw[p] = base + 1;
            } else if (pay[0] == 2) {
              if (!packed_header_ok(pay, len, n, ctl.last[p])) s_bad |= kIlvErrHeader;
              s_raw[p] = base + kPackedHeadBytes;
              ctl.packed[p] = 1;
            } else if (pay[0] == 1 && len >= 5 && ld_u32le(pay + 1) == n) {
              s_coded[p] = 1;
              const uint32_t avail = (uint32_t)(len < 4 * kIlvHeadWords ? len : 4 * kIlvHeadWords);
              ctl.hdr_avail[p] = avail - 5;
              uint64_t tb, dt;
              if (!coded_layout(pay, avail, len, nb, tb, dt)) {
                s_bad |= kIlvErrHeader;
              } else {
                // tab[0] == 0 and tab[nb] == datalen are checked by the
                // wavefronts of the first and last block
                s_table[p] = base + tb;
                s_data[p] = base + dt;
                s_datalen[p] = len - dt;
              }
            } else {
              s_bad |= kIlvErrHeader;
            }
          }
          // table slots of the coded planes, from the last plane down (the
          // exponent plane of the IEEE chains takes slot 0)
          uint32_t k = 0;
          for (uint32_t p = NP; p-- > 0;) {
            ctl.slot[p] = k;
            if (!s_coded[p]) continue;
            if (k < n_slots) {
              ++k;
            } else {  // no table for it in this launch: the tensor is decoded again
              s_coded[p] = 0;
              s_bad |= kIlvRetrySlots;
            }
          }
        }
        __syncthreads();
        // (the build's barriers do not wait for global loads)
        const bool touched = !s_bad && bi < nb;
        if (touched) touch();
#pragma unroll 1
        for (uint32_t p = 0; p < NP; ++p) {
          if (!s_coded[p]) continue;
          // no global loads here: they would wait for the touches (in order)
          uint16_t* tab16 = reinterpret_cast<uint16_t*>(smem + ctl.slot[p] * SLOT);
          const uint8_t* pay = reinterpret_cast<const uint8_t*>(head[p]);
          build_tables(tab16, ctl.t64[p], chain_slot_bytes(C) == kIlvPairLutBytes, ChainInfo<C>::xf[p], bs, pay + 5,
                       ctl.hdr_avail[p]);
          if (t == 0) {
            s_pair[p] = bs.pair;
            if (bs.err) s_bad |= kIlvErrHeader;
          }
          __syncthreads();
        }
        if (touched) {  // the touches complete here
#pragma unroll
          for (uint32_t p = 0; p < NP; ++p) asm volatile("" ::"v"(e_touch[p][0]), "v"(e_touch[p][1]));
        }
        if (t == 0 && s_bad) status_or(&status[ti], s_bad);
      }
      if (s_bad) return;  // uniform: the tensor is rejected
      if (bi >= nb) return;
      if (!prepped) prep();
      if (!ok) {
        bad |= kIlvErrBlock;
        return;
      }
#pragma unroll
      for (uint32_t p = 0; p < NP; ++p)
        if ((st.coded_mask >> p) & 1u && __builtin_amdgcn_readfirstlane(s_pair[p])) st.pair_mask |= 1u << p;
      const uint64_t bstart = (uint64_t)bi * kIlvBlock;
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
      uint32_t q0[NP];
      const bool crc_on = kCrc && T.crc_first != kIlvNoCrc && bstart + kIlvBlock <= n;
      uint32_t acc[NP];
#pragma unroll
      for (uint32_t p = 0; p < NP; ++p) acc[p] = 0;
      // skew uniform planes only when the staging budget has room for it
      if (need + need_skew > stage_words) uni_mask = 0;
      if (need <= stage_words) {
        // Coalesced copy of the block's lane streams into this wavefront's LDS
        // region.  When every lane holds the same number of words c (a
        // fixed-length code, e.g. a uniform nibble plane: 32 words per lane),
        // lane j's stream goes to word (c + skew) j with c + skew odd; left
        // contiguous, all 64 lanes' windows would fall into gcd(c, 64) banks.
        __builtin_amdgcn_wave_barrier();
        uint32_t base = 4;
#pragma unroll
        for (uint32_t p = 0; p < NP; ++p) {
          q0[p] = 0;
          if (!(st.coded_mask & (1u << p))) continue;
          const uint32_t* src = st.words[p];
          uint32_t* dst = sw + base;
          const uint32_t c0 = __builtin_amdgcn_readfirstlane(lane_c[p]);
          const bool uniform = (uni_mask >> p) & 1u;
          const uint32_t skew = uniform ? ((c0 & 1u) ? 2u : 1u) : 0u;
          // words i .. i + 3 (those below tot) to their staging positions
          auto put = [&](uint32_t i, const uint32_t (&x)[4]) {
            if (!uniform) {
              if (i + 4 <= tot[p]) {
                *reinterpret_cast<u32x4*>(dst + i) = u32x4_make(x[0], x[1], x[2], x[3]);
              } else {
                for (uint32_t k = i; k < tot[p]; ++k) dst[k] = x[k - i];
              }
            } else {
              // lane of word i: i / c0 (float estimate, then exact correction);
              // c0 >= 4, so the four words span at most two lanes
              uint32_t j0 = (uint32_t)((float)i * __builtin_amdgcn_rcpf((float)c0));
              if (j0 * c0 > i) --j0;
              if ((j0 + 1) * c0 <= i) ++j0;
              const uint32_t bnd = (j0 + 1) * c0;
#pragma unroll
              for (uint32_t d = 0; d < 4; ++d) {
                const uint32_t w = i + d;
                if (w < tot[p]) dst[w + skew * (j0 + (w >= bnd ? 1u : 0u))] = x[d];
              }
            }
          };
          uint32_t i = 4 * lane;
          for (; i < tot[p]; i += 256) {
            uint32_t x[4] = {0, 0, 0, 0};
            if (i + 4 <= tot[p]) {
              const u32x4a4 v4 = gload_u32x4(src + i);
              x[0] = v4.x;
              x[1] = v4.y;
              x[2] = v4.z;
              x[3] = v4.w;
            } else {
              for (uint32_t k = i; k < tot[p]; ++k) x[k - i] = gload_u32(src + k);
            }
            put(i, x);
          }
          st.q[p] = lds_addr(dst + first[p] + skew * lane) * 8u - 1u;
          q0[p] = st.q[p];
          base += (tot[p] + (uniform ? 128u : 0u) + 3u) & ~3u;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // the bf16 exponent-coded plane forms get a branch-free round body
        const bool fix = C == kChainIeee16Split2 && st.coded_mask == 2u && st.pair_mask == 0u &&
                         st.packed_mask == 0u;
        if (full && crc_on) {
          if (fix) decode_block<C, false, true, kCrc, 3>(st, luts, out, n, bstart, lane, acc);
          else decode_block<C, false, true, kCrc>(st, luts, out, n, bstart, lane, acc);
        } else if (full) {
          if (fix) decode_block<C, false, true, false, 3>(st, luts, out, n, bstart, lane);
          else decode_block<C, false, true, false>(st, luts, out, n, bstart, lane);
        } else if (crc_on) {
          decode_block<C, true, true, kCrc>(st, luts, out, n, bstart, lane, acc);
        } else {
          decode_block<C, true, true, false>(st, luts, out, n, bstart, lane);
        }
        __builtin_amdgcn_wave_barrier();
      } else {
#pragma unroll
        for (uint32_t p = 0; p < NP; ++p) {
          if (st.words[p]) st.words[p] += first[p];
          st.nw[p] = lane_c[p];
          q0[p] = 0;
        }
        if (crc_on) decode_block<C, true, false, kCrc>(st, luts, out, n, bstart, lane, acc);
        else decode_block<C, true, false, false>(st, luts, out, n, bstart, lane);
      }
      if constexpr (kCrc) {
        if (crc_on) {
          // lane l's last piece ends 16 (63 - l) bytes before the block's end
          const uint32_t K = crc_tab[kCrcTabK64 + lane];
#pragma unroll
          for (uint32_t p = 0; p < NP; ++p) {
            uint32_t a = gf2_mulmod_seq(acc[p], K);
#pragma unroll
            for (int d = 32; d >= 1; d >>= 1) a ^= __shfl_xor(a, d, 64);
            if (lane == 0) g_st<uint32_t>(reinterpret_cast<uint64_t>(crc_part + 4ull * (T.crc_first + bi) + p), a);
          }
        }
      }
      // acceptance: every lane's words hold exactly its codes
#pragma unroll
      for (uint32_t p = 0; p < NP; ++p) {
        if (!(st.coded_mask & (1u << p))) continue;
        const uint32_t used = st.q[p] - q0[p];
        if ((used + 31u) / 32u != lane_c[p]) bad |= kIlvErrLane;
      }
    };
    if constexpr (ilv_is_pair(kChain)) {
      if (T.chain == ilv_pair_a(kChain)) body(ChainTag<ilv_pair_a(kChain)>{});
      else body(ChainTag<ilv_pair_b(kChain)>{});
    } else {
      body(ChainTag<kChain>{});
    }
  }
  bad = wave_or_status(bad);
  if (bad && lane == 0) status_or(&status[cur], bad);
}

// ---------------------------------------------------------------------------
// encode kernels
// ---------------------------------------------------------------------------

// Histogram of plane blockIdx.y.  16 LDS copies per workgroup, lane l
// counting into copy l % 16, laid out [symbol][17] so that lanes adding the
// same symbol hit different banks: a skewed plane (an exponent plane has a
// handful of common values) then costs at most four-way conflicts per
// atomic instead of 64.
constexpr uint32_t kHistCopies = 16, kHistStride = 17;

__global__ void __launch_bounds__(256) ilv_hist_kernel(const IlvEncPlane* __restrict__ planes,
                                                       uint32_t* __restrict__ hist) {
  __shared__ uint32_t h[256 * kHistStride];
  const IlvEncPlane P = planes[blockIdx.y];
  const uint32_t t = threadIdx.x, copy = t % kHistCopies;
  for (uint32_t i = t; i < 256 * kHistStride; i += 256) h[i] = 0;
  __syncthreads();
  const uint64_t nvec = P.n / 16;
  const uint64_t stride = (uint64_t)gridDim.x * 256u;
  for (uint64_t v = (uint64_t)blockIdx.x * 256u + t; v < nvec; v += stride) {
    const u32x4 x = gload_nt16(P.src + 16 * v);
    const uint32_t xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int b = 0; b < 4; ++b) atomicAdd(&h[((xs[k] >> (8 * b)) & 0xFFu) * kHistStride + copy], 1u);
  }
  if (blockIdx.x == 0)
    for (uint64_t i = nvec * 16 + t; i < P.n; i += 256) atomicAdd(&h[gload_u8(P.src + i) * kHistStride + copy], 1u);
  __syncthreads();
  uint32_t s = 0;
#pragma unroll
  for (uint32_t c = 0; c < kHistCopies; ++c) s += h[t * kHistStride + c];
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
  const uint64_t bstart = (uint64_t)B.block * kIlvBlock;
  uint32_t bits = 0;
  for (uint32_t r = 0; r < kIlvRounds; ++r) {
    const uint64_t pos = bstart + (uint64_t)kIlvGroup * (r * 64u + lane);
    if (pos >= P.n) continue;
    if (P.n - pos >= kIlvGroup) {
      const u32x4 x = gload_nt16(P.src + pos);
      const uint32_t xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int b = 0; b < 4; ++b) bits += len[(xs[k] >> (8 * b)) & 0xFF];
    } else {
      for (uint64_t k = pos; k < P.n; ++k) bits += len[gload_u8(P.src + k)];
    }
  }
  const uint32_t words = (bits + 31) / 32;
  lane_words[64ull * blockIdx.x + lane] = (uint8_t)words;
  uint32_t incl = wave_incl_scan(words);
  if (lane == 63) block_bytes[blockIdx.x] = 64u + 4u * incl;
}

// One wavefront per block: write lane word counts and packed lane streams.
__device__ __forceinline__ void put_word(bool staged, uint32_t* sw, uint64_t w, uint32_t wi, uint32_t v) {
  if (staged) sw[wi] = v;
  else g_st<uint32_t>(w + 4ull * wi, v);
}

// A block whose coded words (sum of the lane counts) fit stage_words is
// assembled in LDS and written out by the whole wavefront in consecutive
// words; lanes writing their own streams directly scatter 4-byte stores over
// the block (each lane's stream is a different part of it).
__global__ void __launch_bounds__(64) ilv_encode_kernel(const IlvEncPlane* __restrict__ planes,
                                                        const IlvEncBlock* __restrict__ blocks,
                                                        const uint32_t* __restrict__ codes,
                                                        const uint8_t* __restrict__ lane_words,
                                                        uint32_t stage_words) {
  __shared__ uint32_t code[256];
  extern __shared__ uint32_t sbuf[];
  const IlvEncBlock B = blocks[blockIdx.x];
  const IlvEncPlane P = planes[B.plane];
  const uint32_t lane = threadIdx.x;
  for (uint32_t i = lane; i < 256; i += 64) code[i] = codes[256u * P.code_slot + i];
  __syncthreads();
  const uint32_t c = lane_words[64ull * B.lw + lane];
  gstore_u8(B.dst + lane, c);
  const uint32_t incl = wave_incl_scan(c);
  const uint64_t w = B.dst + 64 + 4ull * (incl - c);  // this lane's words
  const uint32_t total = __shfl(incl, 63, 64);
  const bool staged = total <= stage_words;           // uniform
  uint32_t* const sw = sbuf + (incl - c);
  const uint64_t bstart = (uint64_t)B.block * kIlvBlock;
  uint64_t acc = 0;
  uint32_t cnt = 0, wi = 0;
  // (wi < c: the size pass counted these words; the bound only guards a
  // source that changed between the passes)
  // whole groups: one 16-byte load (planes are 16-byte aligned), issued one
  // round ahead; the 16 code lookups issued together
  u32x4 nxt = u32x4_make(0, 0, 0, 0);
  if (bstart + (uint64_t)kIlvGroup * lane + kIlvGroup <= P.n) nxt = gload_nt16(P.src + bstart + (uint64_t)kIlvGroup * lane);
  for (uint32_t r = 0; r < kIlvRounds; ++r) {
    const uint64_t pos = bstart + (uint64_t)kIlvGroup * (r * 64u + lane);
    if (pos >= P.n) continue;
    if (pos + kIlvGroup <= P.n) {
      const u32x4 x = nxt;
      const uint64_t pn = pos + (uint64_t)kIlvGroup * 64u;
      if (r + 1 < kIlvRounds && pn + kIlvGroup <= P.n) nxt = gload_nt16(P.src + pn);
      uint32_t e[kIlvGroup];
#pragma unroll
      for (uint32_t k = 0; k < kIlvGroup; ++k) e[k] = code[(x[k >> 2] >> (8 * (k & 3))) & 0xFFu];
#pragma unroll
      for (uint32_t k = 0; k < kIlvGroup; ++k) {
        acc |= (uint64_t)(e[k] & 0xFFFFu) << cnt;
        cnt += e[k] >> 16;
        if (cnt >= 32) {
          if (wi < c) put_word(staged, sw, w, wi, (uint32_t)acc);
          ++wi;
          acc >>= 32;
          cnt -= 32;
        }
      }
      continue;
    }
    // the plane's partial last group: byte loads
    uint32_t xs[4] = {0, 0, 0, 0};
    const uint32_t count = (uint32_t)(P.n - pos);
    for (uint32_t k = 0; k < count; ++k) xs[k >> 2] |= gload_u8(P.src + pos + k) << (8 * (k & 3));
    for (uint32_t k = 0; k < count; ++k) {
      const uint32_t e = code[(xs[k >> 2] >> (8 * (k & 3))) & 0xFFu];
      acc |= (uint64_t)(e & 0xFFFFu) << cnt;
      cnt += e >> 16;
      if (cnt >= 32) {
        if (wi < c) put_word(staged, sw, w, wi, (uint32_t)acc);
        ++wi;
        acc >>= 32;
        cnt -= 32;
      }
    }
  }
  if (cnt && wi < c) put_word(staged, sw, w, wi, (uint32_t)acc);
  if (staged) {
    __syncthreads();  // one wavefront: its LDS writes are visible to every lane
    for (uint32_t i = lane; i < total; i += 64) g_st<uint32_t>(B.dst + 64 + 4ull * i, sbuf[i]);
  }
}

size_t ilv_decode_lds_bytes(uint32_t chain, uint32_t n_slots, uint32_t stage_words, bool crc) {
  return (size_t)n_slots * chain_slot_bytes(chain) + sizeof(DecodeCtl) +
         (4ull * stage_words + kIlvStageSpare + (crc ? kIlvCrcWords : 0u)) * 4ull;
}

// the fused plane CRC exists for the chains whose plane bytes are the
// decoded symbols up to a byte rotation (crc_chain_supported)
static bool ilv_crc_chain(uint32_t chain) {
  return chain == kChainIeee16Split2 || chain == kChainIeee32Split4 || chain == kChainPassthrough;
}

static const void* ilv_decode_fn(uint32_t chain, bool crc) {
  if (crc) {
    switch (chain) {
      case kChainIeee16Split2: return reinterpret_cast<const void*>(&ilv_decode_kernel<kChainIeee16Split2, true>);
      case kChainIeee32Split4: return reinterpret_cast<const void*>(&ilv_decode_kernel<kChainIeee32Split4, true>);
      case kChainPassthrough: return reinterpret_cast<const void*>(&ilv_decode_kernel<kChainPassthrough, true>);
      default: return nullptr;
    }
  }
  switch (chain) {
    case kChainIeee16Split2: return reinterpret_cast<const void*>(&ilv_decode_kernel<kChainIeee16Split2, false>);
    case kChainIeee32Split4: return reinterpret_cast<const void*>(&ilv_decode_kernel<kChainIeee32Split4, false>);
    case kChainE4m3Nibble: return reinterpret_cast<const void*>(&ilv_decode_kernel<kChainE4m3Nibble, false>);
    case kChainE5m2Nibble: return reinterpret_cast<const void*>(&ilv_decode_kernel<kChainE5m2Nibble, false>);
    case kChainNibbleSplit: return reinterpret_cast<const void*>(&ilv_decode_kernel<kChainNibbleSplit, false>);
    case kChainPassthrough: return reinterpret_cast<const void*>(&ilv_decode_kernel<kChainPassthrough, false>);
    case kIlvPairNibblePass: return reinterpret_cast<const void*>(&ilv_decode_kernel<kIlvPairNibblePass, false>);
    default: return nullptr;
  }
}

hipError_t ilv_decode_occupancy(uint32_t chain, uint32_t n_slots, uint32_t stage_words, bool crc, int* wg_per_cu) {
  const void* fn = ilv_decode_fn(chain, crc);
  if (!fn) return hipErrorInvalidValue;
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(wg_per_cu, fn, 256,
                                                      ilv_decode_lds_bytes(chain, n_slots, stage_words, crc));
}

hipError_t launch_ilv_decode(uint32_t chain, const IlvTensor* tensors, const uint32_t* tix, const uint32_t* tpre,
                             uint32_t m, const IlvInline& inl_in, uint32_t grid, uint32_t* status, uint32_t n_slots,
                             uint32_t stage_words, const uint32_t* crc_tab, uint32_t* crc_part, hipStream_t stream) {
  if (!grid || !(inl_in.m ? inl_in.m : m)) return hipSuccess;
  if (inl_in.m > kIlvInlineTensors) return hipErrorInvalidValue;
  IlvInline inl = inl_in;
  if (stage_words % 4 != 0 || stage_words < 8) return hipErrorInvalidValue;
  const bool crc = crc_tab != nullptr;
  if (crc && (!crc_part || !ilv_crc_chain(chain))) return hipErrorInvalidValue;
  const size_t lds = ilv_decode_lds_bytes(chain, n_slots, stage_words, crc);
  const void* fn = ilv_decode_fn(chain, crc);
  if (!fn) return hipErrorInvalidValue;
  void* args[] = {&inl, &tensors, &tix, &tpre, &m, &status, &n_slots, &stage_words, &crc_tab, &crc_part};
  const hipError_t e = hipLaunchKernel(fn, dim3(grid), dim3(256), args, lds, stream);
  return e != hipSuccess ? e : hipGetLastError();
}

// Packed-nibble payload bodies: job blockIdx.y, each thread turns 16 plane
// bytes (symbols < 16) into 8 output bytes, byte i = s[2i] | s[2i+1] << 4.
// The thread whose vector index is n / 16 packs the tail.
__device__ __forceinline__ uint32_t pack_nibbles4(uint32_t w) {
  // bytes s0 s1 s2 s3 -> (s0 | s1 << 4) | (s2 | s3 << 4) << 8
  const uint32_t t = (w & 0x000F000Fu) | ((w >> 4) & 0x00F000F0u);
  return (t & 0xFFu) | ((t >> 8) & 0xFF00u);
}

__global__ void __launch_bounds__(256) ilv_pack_kernel(const IlvPackJob* __restrict__ jobs) {
  const IlvPackJob J = jobs[blockIdx.y];
  const uint64_t nvec = J.n / 16;
  const uint64_t stride = (uint64_t)gridDim.x * 256u;
  for (uint64_t v = (uint64_t)blockIdx.x * 256u + threadIdx.x; v <= nvec; v += stride) {
    if (v < nvec) {
      const u32x4 x = gload_nt16(J.src + 16 * v);
      const uint32_t lo = pack_nibbles4(x.x) | (pack_nibbles4(x.y) << 16);
      const uint32_t hi = pack_nibbles4(x.z) | (pack_nibbles4(x.w) << 16);
      const uint64_t w = (uint64_t)lo | ((uint64_t)hi << 32);
      if ((J.dst & 7u) == 0) {
        g_st<uint64_t>(J.dst + 8 * v, w);
      } else {  // output buffer not 8-byte aligned
        for (int k = 0; k < 8; ++k) gstore_u8(J.dst + 8 * v + k, (uint32_t)(w >> (8 * k)) & 0xFFu);
      }
    } else {
      for (uint64_t i = 16 * nvec; i < J.n; i += 2) {
        uint32_t b = gload_u8(J.src + i) & 0xFu;
        if (i + 1 < J.n) b |= (gload_u8(J.src + i + 1) & 0xFu) << 4;
        gstore_u8(J.dst + i / 2, b);
      }
    }
  }
}

// Job blockIdx.y; output vector v = bytes [16 v, 16 v + 16) of the payload
// body at dst (shift 1: body byte 0 is the tag, byte k + 1 plane byte k).
// The thread past the last whole output vector writes the tail bytewise.
__global__ void __launch_bounds__(256) ilv_store_kernel(const IlvStoreJob* __restrict__ jobs) {
  const IlvStoreJob J = jobs[blockIdx.y];
  const uint64_t out_n = J.n + J.shift;
  const uint64_t nvec = out_n / 16;
  const uint64_t stride = (uint64_t)gridDim.x * 256u;
  const bool aligned = (J.dst & 15u) == 0;
  for (uint64_t v = (uint64_t)blockIdx.x * 256u + threadIdx.x; v <= nvec; v += stride) {
    if (v < nvec) {
      // plane bytes [16 v - shift, 16 v + 16 - shift); the 16-byte aligned
      // load at 16 v starts inside the plane (16 v < n)
      const u32x4 x = gload_nt16(J.src + 16 * v);
      u32x4 o = x;
      if (J.shift) {
        const uint32_t prev = v == 0 ? 0u : gload_u8(J.src + 16 * v - 1);  // tag 0 before plane byte 0
        o = u32x4_make((x.x << 8) | prev, __builtin_amdgcn_alignbit(x.y, x.x, 24),
                       __builtin_amdgcn_alignbit(x.z, x.y, 24), __builtin_amdgcn_alignbit(x.w, x.z, 24));
      }
      if (aligned) {
        g_st<u32x4>(J.dst + 16 * v, o);
      } else {
        for (int k = 0; k < 16; ++k) gstore_u8(J.dst + 16 * v + k, o[k >> 2] >> (8 * (k & 3)));
      }
    } else {
      for (uint64_t i = 16 * nvec; i < out_n; ++i)
        gstore_u8(J.dst + i, i < J.shift ? 0u : gload_u8(J.src + i - J.shift));
    }
  }
}

// Realigned copies of coded payloads (any source alignment) to 16-byte
// aligned scratch: per 16 output bytes, the five source dwords that hold
// them, shifted into place with alignbyte.  A source dword is read only if
// it starts before the payload's end, so no read leaves the dword that holds
// the payload's last byte.
__global__ void __launch_bounds__(256) ilv_realign_kernel(const IlvStoreJob* __restrict__ jobs) {
  const IlvStoreJob J = jobs[blockIdx.y];
  const uint64_t nvec = (J.n + 15) / 16, end = J.src + J.n;
  const uint64_t stride = (uint64_t)gridDim.x * 256u;
  for (uint64_t v = (uint64_t)blockIdx.x * 256u + threadIdx.x; v < nvec; v += stride) {
    const uint64_t s = J.src + 16 * v, a = s & ~3ull;
    const uint32_t sh = (uint32_t)(s & 3u);
    uint32_t w[5];
#pragma unroll
    for (int k = 0; k < 5; ++k) w[k] = a + 4u * k < end ? g_ld<uint32_t>(a + 4u * k) : 0u;
    const u32x4 o = u32x4_make(__builtin_amdgcn_alignbyte(w[1], w[0], sh), __builtin_amdgcn_alignbyte(w[2], w[1], sh),
                               __builtin_amdgcn_alignbyte(w[3], w[2], sh), __builtin_amdgcn_alignbyte(w[4], w[3], sh));
    if (16 * v + 16 <= J.n) {
      g_st<u32x4>(J.dst + 16 * v, o);
    } else {
      for (uint64_t k = 16 * v; k < J.n; ++k) gstore_u8(J.dst + k, o[(k - 16 * v) >> 2] >> (8 * ((k - 16 * v) & 3)));
    }
  }
}

hipError_t launch_ilv_realign(const IlvStoreJob* jobs, uint32_t n_jobs, uint64_t max_n, hipStream_t stream) {
  if (!n_jobs) return hipSuccess;
  uint64_t blocks = (max_n / 16 + 256) / 256;
  if (blocks > 1024) blocks = 1024;
  for (uint32_t j0 = 0; j0 < n_jobs; j0 += kMaxGridY) {
    const uint32_t cnt = n_jobs - j0 < kMaxGridY ? n_jobs - j0 : kMaxGridY;
    hipLaunchKernelGGL(ilv_realign_kernel, dim3((uint32_t)blocks, cnt), dim3(256), 0, stream, jobs + j0);
  }
  return hipGetLastError();
}

hipError_t launch_ilv_store(const IlvStoreJob* jobs, uint32_t n_jobs, uint64_t max_n, hipStream_t stream) {
  if (!n_jobs) return hipSuccess;
  uint64_t blocks = (max_n / 16 + 256) / 256;
  if (blocks > 1024) blocks = 1024;
  // gridDim.y is at most 65535: slices of jobs
  for (uint32_t j0 = 0; j0 < n_jobs; j0 += kMaxGridY) {
    const uint32_t cnt = n_jobs - j0 < kMaxGridY ? n_jobs - j0 : kMaxGridY;
    hipLaunchKernelGGL(ilv_store_kernel, dim3((uint32_t)blocks, cnt), dim3(256), 0, stream, jobs + j0);
  }
  return hipGetLastError();
}

hipError_t launch_ilv_pack(const IlvPackJob* jobs, uint32_t n_jobs, uint64_t max_n, hipStream_t stream) {
  if (!n_jobs) return hipSuccess;
  uint64_t blocks = (max_n / 16 + 256) / 256;
  if (blocks > 1024) blocks = 1024;
  for (uint32_t j0 = 0; j0 < n_jobs; j0 += kMaxGridY) {
    const uint32_t cnt = n_jobs - j0 < kMaxGridY ? n_jobs - j0 : kMaxGridY;
    hipLaunchKernelGGL(ilv_pack_kernel, dim3((uint32_t)blocks, cnt), dim3(256), 0, stream, jobs + j0);
  }
  return hipGetLastError();
}

hipError_t launch_ilv_hist(const IlvEncPlane* planes, uint32_t n_planes, uint64_t max_n, uint32_t* hist,
                           hipStream_t stream) {
  if (!n_planes) return hipSuccess;
  uint64_t blocks = (max_n / 16 + 255) / 256;
  if (blocks > 512) blocks = 512;
  if (blocks < 1) blocks = 1;
  for (uint32_t p0 = 0; p0 < n_planes; p0 += kMaxGridY) {
    const uint32_t cnt = n_planes - p0 < kMaxGridY ? n_planes - p0 : kMaxGridY;
    hipLaunchKernelGGL(ilv_hist_kernel, dim3((uint32_t)blocks, cnt), dim3(256), 0, stream, planes + p0,
                       hist + 256ull * p0);
  }
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
                             const uint32_t* codes, const uint8_t* lane_words, uint32_t stage_words,
                             hipStream_t stream) {
  if (!n_blocks) return hipSuccess;
  if (stage_words > kIlvEncStageMax) return hipErrorInvalidValue;
  hipLaunchKernelGGL(ilv_encode_kernel, dim3(n_blocks), dim3(64), 4ull * stage_words, stream, planes, blocks, codes,
                     lane_words, stage_words);
  return hipGetLastError();
}

}  // namespace ptwm
