// zstd_device.hip -- Zstandard frames, the reference's Zstd plane codec
// (codecs/zstd.rs -> the zstd crate's decode_all, codec_tagged.rs:198-307),
// decoded on gfx950.
//
// One 64-lane workgroup per payload (a plane or one chunk frame), decoding
// RFC 8878 frames in order: frame and block headers, raw and RLE blocks
// (copied by the whole wavefront), and compressed blocks:
//   literals  Huffman tables (direct or FSE-coded weights) built in LDS by
//             the wavefront; the 4 streams decoded by 4 lanes at once, into
//             the tail of the output buffer (see below), or raw / RLE;
//   sequences FSE tables (predefined, RLE, described, repeated) in LDS; the
//             serial state chain and the sequence execution on lane 0.
// The decoded literals of a block live in the last `regen` bytes of the
// output: the block's literals are all emitted, so the write position stays
// at or below the next unread literal (checked for every sequence), and no
// literal buffer is needed.  Limits and rejections follow libzstd 1.5.7's
// decoder, which the reference links: window above 2^27 + 1 bytes, a
// dictionary id, weights above 12, fewer than 6 literals in 4-stream mode,
// an unconsumed bitstream, offsets before the frame's start.  The decoded
// length must equal the job's (the chunk table's / the plane's).
#include "decode_sync.h"
#include "ptwm_common.h"

namespace ptwm {

namespace {

constexpr uint32_t kZBlockMax = 128u * 1024u;
constexpr uint32_t kZBatch = 96;                // sequences decoded per batch
// LDS: about 23 KB a workgroup, so seven payloads decode on a CU at once
constexpr uint32_t kZRing = 2u * 1024u;         // LDS history ring (bytes)
constexpr uint32_t kZLitStage = 1u * 1024u;     // literal bytes of a batch staged in LDS
constexpr uint32_t kZSeqStage = 288;             // sequence stream words staged per batch
constexpr uint32_t kZHufMax = 12;

// code tables of RFC 8878 3.1.1.3.2.1 and default distributions 3.1.1.3.2.2
__constant__ uint32_t kLLBase[36] = {0,  1,  2,  3,  4,  5,  6,   7,   8,   9,   10,   11,   12,   13,    14,    15,   16,   18,
                                     20, 22, 24, 28, 32, 40, 48, 64, 128, 256, 512, 1024, 2048, 4096, 8192, 16384, 32768, 65536};
__constant__ uint8_t kLLBits[36] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 1, 1,
                                    1, 1, 2, 2, 3, 3, 4, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16};
__constant__ uint32_t kMLBase[53] = {3,  4,  5,  6,  7,  8,  9,  10,  11,  12,  13,  14,   15,   16,   17,   18,   19,    20,
                                     21, 22, 23, 24, 25, 26, 27, 28,  29,  30,  31,  32,   33,   34,   35,   37,   39,    41,
                                     43, 47, 51, 59, 67, 83, 99, 131, 259, 515, 1027, 2051, 4099, 8195, 16387, 32771, 65539};
__constant__ uint8_t kMLBits[53] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0,
                                    0, 0, 0, 0, 0, 1, 1, 1, 1, 2, 2, 3, 3, 4, 4, 5, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16};
__constant__ int16_t kLLDef[36] = {4, 3, 2, 2, 2, 2, 2, 2, 2, 2, 2, 2, 2, 1, 1, 1, 2, 2,
                                   2, 2, 2, 2, 2, 2, 2, 3, 2, 1, 1, 1, 1, 1, -1, -1, -1, -1};
__constant__ int16_t kMLDef[53] = {1, 4, 3, 2, 2, 2, 2, 2, 2, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1,
                                   1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, -1, -1, -1, -1, -1, -1, -1};
__constant__ int16_t kOFDef[29] = {1, 1, 1, 1, 1, 1, 2, 2, 2, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, -1, -1, -1, -1, -1};

__device__ __forceinline__ uint32_t zld8(const uint8_t* p) { return g_ld<uint8_t>((uint64_t)p); }
__device__ __forceinline__ uint32_t hibit(uint32_t x) { return 31u - (uint32_t)__builtin_clz(x); }

// Backward bit reader (RFC 8878 4.1 / 4.2.2): `pos` = real bits not yet read;
// reading nb bits takes stream bits [pos - nb, pos) as a little-endian
// integer (zeros below bit 0) and lowers pos, which may go negative.
// The stream is read as aligned 32-bit words (a word holding a stream byte
// never crosses a page); bit positions count from the first aligned word
// (stream bit 0 is bit 8 a, a = the stream's address mod 4).  A 64-bit
// window holds bits [32 wi, 32 wi + 64) with rel = pos + 8 a - 32 wi in
// [32, 64] between reads; when a read leaves fewer than 32 bits in it, the
// next lower word, loaded one refill earlier, is shifted in.  Bits below
// the stream (before its first byte, or below word 0) read as zero.
struct ZBits {
  uint64_t base;   // the stream's address rounded down to 4
  uint32_t lead;   // 8 a: bits of word 0 before the stream
  uint32_t rel;
  int64_t wi;
  uint64_t w;
  uint32_t nx;     // word wi - 1 as loaded (word 0 when wi - 1 < 0)
  int32_t sw;      // sequence reader: wi's index in the LDS stage
};

__device__ __forceinline__ uint32_t zb_load(const ZBits& b, int64_t k) {
  return g_ld<uint32_t>(b.base + 4ull * (uint64_t)(k < 0 ? 0 : k));
}
// word k as the window takes it: zero below the stream
__device__ __forceinline__ uint32_t zb_take(const ZBits& b, int64_t k, uint32_t v) {
  if ((int32_t)((uint64_t)k >> 32) < 0) return 0u;  // k < 0
  return k == 0 ? v & ~((1u << b.lead) - 1u) : v;  // lead < 32
}

__device__ bool zb_init(ZBits& b, const uint8_t* p, uint64_t n) {
  if (n == 0) return false;
  const uint32_t last = zld8(p + n - 1);
  if (!last) return false;
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  b.base = a & ~3ull;
  b.lead = 8u * (uint32_t)(a & 3u);
  const int64_t pa = (int64_t)(n * 8) - (int64_t)(8 - hibit(last)) + b.lead;  // >= lead >= 0
  const int64_t top = (pa - 1) >> 5;  // word holding bit pa - 1 (-1 when pa == 0)
  b.wi = top - 1;
  b.w = ((uint64_t)zb_take(b, top, zb_load(b, top)) << 32) | zb_take(b, top - 1, zb_load(b, top - 1));
  b.nx = zb_load(b, top - 2);
  b.rel = (uint32_t)(pa - 32 * b.wi);  // in [33, 64]
  return true;
}

__device__ __forceinline__ int64_t zb_pos(const ZBits& b) { return 32 * b.wi + (int64_t)b.rel - (int64_t)b.lead; }

// nb <= 32
__device__ __forceinline__ uint32_t zb_peek(const ZBits& b, uint32_t nb) {
  return nb == 0 ? 0u : (uint32_t)((b.w >> (b.rel - nb)) & ((1ull << nb) - 1ull));
}

__device__ __forceinline__ void zb_skip(ZBits& b, uint32_t nb) {
  b.rel -= nb;
  if (b.rel < 32) {
    b.w = (b.w << 32) | zb_take(b, b.wi - 1, b.nx);
    b.rel += 32;
    --b.wi;
    b.nx = zb_load(b, b.wi - 1);
  }
}

__device__ __forceinline__ uint32_t zb_read(ZBits& b, uint32_t nb) {
  const uint32_t v = zb_peek(b, nb);
  zb_skip(b, nb);
  return v;
}

// The sequence stream's reader takes its words from an LDS stage instead:
// before each batch the wavefront stages the kZSeqStage words below the
// window (a batch reads at most kZBatch x 90 bits), and a refill reads the
// next lower word from there; the word read at one refill is made
// wave-uniform at the next, so the LDS read is not waited for in between.
__device__ __forceinline__ void zs_skip(ZBits& b, uint32_t nb, const uint32_t* stage) {
  b.rel -= nb;
  if (b.rel < 32) {
    b.w = (b.w << 32) | zb_take(b, b.wi - 1, (uint32_t)__builtin_amdgcn_readfirstlane(b.nx));
    b.rel += 32;
    --b.wi;
    --b.sw;
    b.nx = b.sw >= 1 ? stage[b.sw - 1] : 0u;
  }
}
// nb bits with no refill (the caller keeps rel >= nb)
__device__ __forceinline__ uint32_t zs_take(ZBits& b, uint32_t nb) {
  const uint32_t v = zb_peek(b, nb);
  b.rel -= nb;
  return v;
}
// refill once if fewer than 32 bits remain (one refill restores >= 32)
__device__ __forceinline__ void zs_fill(ZBits& b, const uint32_t* stage) { zs_skip(b, 0, stage); }

// a 64-bit value read from LDS, made wave-uniform
__device__ __forceinline__ uint64_t zu64(uint64_t v) {
  return ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32)) << 32) |
         (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
}

// an output byte, to the plane and to the history ring
__device__ __forceinline__ void z_put(uint8_t* dst, uint8_t* ring, uint64_t pos, uint32_t b) {
  g_st<uint8_t>((uint64_t)(dst + pos), (uint8_t)b);
  ring[pos & (kZRing - 1)] = (uint8_t)b;
}

// A match (3.1.1.4) of ml bytes at output position o from off bytes back,
// by the wavefront, 64 bytes an instruction.  Offsets up to the ring's
// size read the LDS ring (the wavefront's LDS accesses complete in order,
// so a chunk sees every earlier chunk); an offset below 64 repeats the last
// off bytes (byte j of the match is byte j mod off of them).  Longer
// offsets read the plane: a chunk whose sources reach bytes stored since
// the last fence fences first; the caller may pass the match's first bytes
// already loaded (pre, pn).
__device__ __forceinline__ void z_match(uint8_t* dst, uint8_t* ring, uint64_t o, uint32_t off, uint32_t ml,
                                        uint32_t lane, uint64_t& fence_o, const uint8_t* pre, uint32_t pn) {
  if (ml == 0) return;
  if (off < 64) {
    uint32_t ph = lane % off;  // (c + lane) mod off for chunk start c
    const uint32_t step = 64u % off;
    for (uint32_t c0 = 0; c0 < ml; c0 += 64) {
      const uint32_t b = ring[(o - off + ph) & (kZRing - 1)];
      if (c0 + lane < ml) z_put(dst, ring, o + c0 + lane, b);
      ph += step;
      if (ph >= off) ph -= off;
    }
  } else if (off <= kZRing) {
    for (uint32_t c0 = 0; c0 < ml; c0 += 64) {
      const uint64_t pos = o + c0 + lane;
      const uint32_t b = ring[(pos - off) & (kZRing - 1)];
      if (c0 + lane < ml) z_put(dst, ring, pos, b);
    }
  } else {
    // the first pn bytes (pn <= 8) were loaded with the batch's other far
    // sources before it ran
    for (uint32_t c0 = 0; c0 < ml; c0 += 64) {
      if (c0 + 64 > pn && ml > pn && o + c0 - off + 64 > fence_o) {
        __threadfence_block();
        fence_o = o + c0;
      }
      const uint64_t pos = o + c0 + lane;
      const uint32_t b = c0 + lane < pn ? (uint32_t)pre[lane] : c0 + lane < ml ? zld8(dst + pos - off) : 0u;
      if (c0 + lane < ml) z_put(dst, ring, pos, b);
    }
  }
}

// forward bit reader over global bytes (FSE table descriptions, 4.1.1)
__device__ uint32_t zf_peek(const uint8_t* p, uint64_t n, uint64_t bit, uint32_t nb) {
  uint32_t v = 0;
  for (uint32_t i = 0; i < nb; ++i) {
    const uint64_t b = bit + i;
    if ((b >> 3) < n) v |= ((zld8(p + (b >> 3)) >> (b & 7)) & 1u) << i;
  }
  return v;
}

// 4.1.1 normalized counts; bytes consumed or -1
__device__ int64_t z_ncount(const uint8_t* p, uint64_t n, uint32_t max_al, uint32_t max_sym, int16_t* norm,
                            uint32_t& al_out, uint32_t& nsym_out) {
  if (n < 1) return -1;
  uint64_t bit = 4;
  const uint32_t al = zf_peek(p, n, 0, 4) + 5;
  if (al > max_al) return -1;
  int32_t remaining = (1 << al) + 1, threshold = 1 << al, nb = (int32_t)al + 1;
  uint32_t s = 0;
  bool prev0 = false;
  while (remaining > 1 && s <= max_sym) {
    if (prev0) {
      uint32_t n0 = s;
      for (;;) {
        if ((bit + 2 + 7) / 8 > n) return -1;
        const uint32_t rep = zf_peek(p, n, bit, 2);
        bit += 2;
        n0 += rep;
        if (rep != 3) break;
      }
      if (n0 > max_sym) return -1;
      while (s < n0) norm[s++] = 0;
    }
    const int32_t mx = (2 * threshold - 1) - remaining;
    int32_t count;
    const uint32_t low = zf_peek(p, n, bit, (uint32_t)nb - 1);
    if ((int32_t)low < mx) {
      count = (int32_t)low;
      bit += (uint64_t)(nb - 1);
    } else {
      count = (int32_t)zf_peek(p, n, bit, (uint32_t)nb);
      if (count >= threshold) count -= mx;
      bit += (uint64_t)nb;
    }
    if ((bit + 7) / 8 > n) return -1;
    count--;
    remaining -= count < 0 ? -count : count;
    norm[s++] = (int16_t)count;
    prev0 = count == 0;
    while (remaining < threshold) {
      nb--;
      threshold >>= 1;
    }
  }
  if (remaining != 1) return -1;
  al_out = al;
  nsym_out = s;
  return (int64_t)((bit + 7) / 8);
}

// 4.1.1 decoding table into t[]: entry = sym | nb << 8 | baseline << 16
__device__ void z_fse_build(uint32_t* t, const int16_t* norm, uint32_t nsym, uint32_t al, uint16_t* next) {
  const uint32_t size = 1u << al;
  uint32_t high = size - 1;
  for (uint32_t s = 0; s < nsym; ++s) {
    if (norm[s] == -1) {
      t[high--] = s;
      next[s] = 1;
    } else {
      next[s] = (uint16_t)norm[s];
    }
  }
  const uint32_t step = (size >> 1) + (size >> 3) + 3, mask = size - 1;
  uint32_t pos = 0;
  for (uint32_t s = 0; s < nsym; ++s)
    for (int32_t i = 0; i < norm[s]; ++i) {
      t[pos] = s;
      do {
        pos = (pos + step) & mask;
      } while (pos > high);
    }
  for (uint32_t u = 0; u < size; ++u) {
    const uint32_t s = t[u] & 255u, x = next[s]++;
    const uint32_t nbits = al - hibit(x);
    t[u] = s | (nbits << 8) | (((x << nbits) - size) << 16);
  }
}

// Per-workgroup state (lane 0 writes, the wavefront reads after a barrier).
enum : uint32_t { kZDone = 0, kZError, kZRaw, kZRle, kZComp };

struct ZCtl {
  uint64_t i, n;        // payload cursor / length (relative to src)
  uint64_t o;           // output bytes written
  uint64_t frame_start;
  uint32_t action;
  uint32_t status;
  uint64_t blk_off, blk_len;  // current block (src offsets)
  uint64_t bmax;
  // literals of the current compressed block
  uint32_t lit_type, regen, n_streams, huf_new, err;
  uint64_t lit_src;           // raw literals: src offset; RLE: the byte
  uint64_t seg_off[4], seg_len[4];
  uint32_t seg_cnt[4];
  uint64_t seq_off;           // sequences section (src offset)
  // frame
  uint32_t in_frame, checksum;
  uint64_t fcs;
  uint32_t fcs_known;
  uint32_t have_huf, have_ll, have_of, have_ml;
  uint32_t rep[3];
  uint32_t huf_bits;
  uint32_t ns;                // Huffman symbols (with the implied last one)
  uint32_t al[3];             // accuracy logs of the LL, OF, ML tables
  uint64_t nseq;              // sequences of the current block
  uint32_t batch, seq_ok;     // sequences in the current batch; no error so far
  uint64_t batch_lits;        // literal bytes the batch copies
  int64_t seq_wi;             // the sequence reader's window word
  uint64_t seq_base;          // the sequence stream's aligned address
  uint64_t seq_w;             // the reader's window, offset and next word
  uint32_t seq_rel, seq_nx, seq_lead;
  uint32_t seq_state[3];      // LL, OF, ML states
};

// XXH64 with seed 0 (the frame checksum), serial on one lane
constexpr uint64_t kX1 = 0x9E3779B185EBCA87ull, kX2 = 0xC2B2AE3D27D4EB4Full, kX3 = 0x165667B19E3779F9ull,
                   kX4 = 0x85EBCA77C2B2AE63ull, kX5 = 0x27D4EB2F165667C5ull;
__device__ __forceinline__ uint64_t xrotl(uint64_t x, int r) { return (x << r) | (x >> (64 - r)); }
__device__ __forceinline__ uint64_t xrd(const uint8_t* p, int k) {
  uint64_t v = 0;
  for (int i = k - 1; i >= 0; --i) v = (v << 8) | zld8(p + i);
  return v;
}
__device__ __forceinline__ uint64_t xround(uint64_t a, uint64_t x) { return xrotl(a + x * kX2, 31) * kX1; }
__device__ uint64_t z_xxh64(const uint8_t* p, uint64_t n) {
  uint64_t h;
  const uint8_t* e = p + n;
  if (n >= 32) {
    uint64_t v1 = kX1 + kX2, v2 = kX2, v3 = 0, v4 = 0 - kX1;
    for (; e - p >= 32; p += 32) {
      v1 = xround(v1, xrd(p, 8));
      v2 = xround(v2, xrd(p + 8, 8));
      v3 = xround(v3, xrd(p + 16, 8));
      v4 = xround(v4, xrd(p + 24, 8));
    }
    h = xrotl(v1, 1) + xrotl(v2, 7) + xrotl(v3, 12) + xrotl(v4, 18);
    h = (h ^ xround(0, v1)) * kX1 + kX4;
    h = (h ^ xround(0, v2)) * kX1 + kX4;
    h = (h ^ xround(0, v3)) * kX1 + kX4;
    h = (h ^ xround(0, v4)) * kX1 + kX4;
  } else {
    h = kX5;
  }
  h += n;
  for (; e - p >= 8; p += 8) h = xrotl(h ^ xround(0, xrd(p, 8)), 27) * kX1 + kX4;
  if (e - p >= 4) {
    h = xrotl(h ^ (xrd(p, 4) * kX1), 23) * kX2 + kX3;
    p += 4;
  }
  for (; p < e; ++p) h = xrotl(h ^ ((uint64_t)zld8(p) * kX5), 11) * kX1;
  h ^= h >> 33;
  h *= kX2;
  h ^= h >> 29;
  h *= kX3;
  h ^= h >> 32;
  return h;
}

}  // namespace

// Huffman weights (4.2.1) of the tree description at p[0..n): lane 0.
// Fills w[0..ns), returns bytes consumed or -1.
__device__ int64_t z_huf_weights(const uint8_t* p, uint64_t n, uint8_t* w, uint32_t& ns, uint32_t& max_bits,
                                 uint32_t* ftab, int16_t* norm, uint16_t* next) {
  if (n < 1) return -1;
  const uint32_t hb = zld8(p);
  uint32_t nw = 0;
  int64_t used;
  if (hb >= 128) {
    nw = hb - 127;
    const uint64_t bytes = (nw + 1) / 2;
    if (1 + bytes > n) return -1;
    for (uint32_t i = 0; i < nw; ++i) {
      const uint32_t b = zld8(p + 1 + i / 2);
      w[i] = (uint8_t)((i % 2 == 0) ? (b >> 4) : (b & 15u));
    }
    used = (int64_t)(1 + bytes);
  } else {
    if (1 + (uint64_t)hb > n) return -1;
    const uint8_t* q = p + 1;
    uint32_t al, nsym;
    const int64_t u = z_ncount(q, hb, 6, 255, norm, al, nsym);
    if (u < 0 || (uint64_t)u > hb) return -1;
    z_fse_build(ftab, norm, nsym, al, next);
    ZBits r;
    if (!zb_init(r, q + u, hb - (uint64_t)u)) return -1;
    uint32_t s1 = zb_read(r, al), s2 = zb_read(r, al);
    // two interleaved states until the stream is over-read (FSE tail loop)
    for (;;) {
      if (nw > 253) return -1;
      w[nw++] = (uint8_t)ftab[s1];
      s1 = (ftab[s1] >> 16) + zb_read(r, (ftab[s1] >> 8) & 255u);
      if (zb_pos(r) < 0) {
        w[nw++] = (uint8_t)ftab[s2];
        break;
      }
      if (nw > 253) return -1;
      w[nw++] = (uint8_t)ftab[s2];
      s2 = (ftab[s2] >> 16) + zb_read(r, (ftab[s2] >> 8) & 255u);
      if (zb_pos(r) < 0) {
        w[nw++] = (uint8_t)ftab[s1];
        break;
      }
    }
    used = (int64_t)(1 + hb);
  }
  // the implied last weight completes a power of two (4.2.1.3)
  uint32_t total = 0;
  for (uint32_t i = 0; i < nw; ++i) {
    if (w[i] > kZHufMax) return -1;
    if (w[i]) total += 1u << (w[i] - 1);
  }
  if (total == 0) return -1;
  const uint32_t mb = hibit(total) + 1;
  const uint32_t rest = (1u << mb) - total;
  if ((rest & (rest - 1)) || mb > kZHufMax || nw + 1 > 256) return -1;
  w[nw] = (uint8_t)(hibit(rest) + 1);
  ns = nw + 1;
  uint32_t r1 = 0;
  for (uint32_t i = 0; i < ns; ++i) r1 += w[i] == 1;
  if (r1 < 2 || (r1 & 1)) return -1;
  max_bits = mb;
  return used;
}

__global__ void __launch_bounds__(64) zstd_decode_kernel(const DecodeJob* __restrict__ jobs,
                                                         uint32_t* __restrict__ status) {
  __shared__ ZCtl c;
  __shared__ uint16_t huf[1u << kZHufMax];  // sym | nb << 8
  __shared__ uint8_t hw[256];               // Huffman weights
  __shared__ uint16_t hstart[256];          // first table slot of each symbol
  __shared__ uint32_t ll_t[512], ml_t[512], of_t[256];
  __shared__ uint32_t ftab[64];             // the weights' FSE table
  __shared__ int16_t norm[256];
  __shared__ uint16_t next[256];
  __shared__ uint32_t sq_ll[kZBatch], sq_ml[kZBatch], sq_off[kZBatch];  // a batch of decoded sequences
  __shared__ uint64_t sq_src[kZBatch];                                  // their match sources
  __shared__ uint8_t sq_pre[8 * kZBatch];                               // first source bytes of far matches
  __shared__ uint8_t ring[kZRing];                                      // the last kZRing output bytes
  __shared__ uint8_t lit_stage[kZLitStage];                             // literals of the current batch
  __shared__ uint32_t seq_stage[kZSeqStage];                            // sequence stream words below the window
  uint64_t fence_o = 0;  // output bytes below this were stored before the last fence

  const DecodeJob job = jobs[blockIdx.x];
  if (job.codec != kCodecZstd) return;
  const uint32_t lane = threadIdx.x;
  // the LL and ML codes (baseline | extra bits << 24), code c in lane c of a
  // register: a sequence step reads its codes with one lane read each
  const uint32_t ll_code = lane < 36 ? kLLBase[lane] | ((uint32_t)kLLBits[lane] << 24) : 0u;
  const uint32_t ml_code = lane < 53 ? kMLBase[lane] | ((uint32_t)kMLBits[lane] << 24) : 0u;
  const uint8_t* src = reinterpret_cast<const uint8_t*>(job.src);
  uint8_t* dst = reinterpret_cast<uint8_t*>(job.dst);
  const uint64_t cap = job.dst_len;

  if (lane == 0) {
    c.status = kStOk;
    c.action = kZDone;
    c.i = 0;
    c.n = job.src_len;
    c.o = 0;
    c.in_frame = 0;
    c.err = 0;
    if (job.framed) {  // chunk frame [ver][state_len u32][state][payload] (container.rs:2010-2049)
      if (c.n < 5) {
        c.status = kStBadFrame;
      } else {
        const uint64_t sl = zld8(src + 1) | (zld8(src + 2) << 8) | (zld8(src + 3) << 16) | ((uint64_t)zld8(src + 4) << 24);
        if (c.n - 5 < sl) c.status = kStBadFrame;
        else c.i = 5 + sl;
      }
    }
  }
  __syncthreads();
  if (c.status != kStOk) {
    if (lane == 0) status[blockIdx.x] = c.status;
    return;
  }

  for (;;) {
    __syncthreads();  // every lane has read the last step's action
    // ---- lane 0: frame / block headers; what the wavefront does next ----
    if (lane == 0) {
      uint32_t act = kZError;
      for (;;) {
        if (!c.in_frame) {
          if (c.i == c.n) {
            act = kZDone;
            break;
          }
          if (c.n - c.i < 4) break;
          const uint8_t* s = src + c.i;
          const uint32_t magic = zld8(s) | (zld8(s + 1) << 8) | (zld8(s + 2) << 16) | (zld8(s + 3) << 24);
          if ((magic & 0xFFFFFFF0u) == 0x184D2A50u) {  // skippable frame (3.1.2)
            if (c.n - c.i < 8) break;
            const uint64_t sz = zld8(s + 4) | (zld8(s + 5) << 8) | (zld8(s + 6) << 16) | ((uint64_t)zld8(s + 7) << 24);
            if (c.n - c.i - 8 < sz) break;
            c.i += 8 + sz;
            continue;
          }
          if (magic != 0xFD2FB528u) break;
          uint64_t i = c.i + 4;
          if (i >= c.n) break;
          const uint32_t fhd = zld8(src + i++);
          const uint32_t fcs_flag = fhd >> 6, single = (fhd >> 5) & 1u, did = fhd & 3u;
          if (fhd & 8u) break;
          uint64_t window = 0;
          if (!single) {
            if (i >= c.n) break;
            const uint32_t wd = zld8(src + i++);
            const uint64_t base = 1ull << (10 + (wd >> 3));
            window = base + (base / 8) * (wd & 7u);
          }
          const uint32_t db = did == 3 ? 4 : did;
          if (c.n - i < db) break;
          uint32_t dict = 0;
          for (uint32_t k = 0; k < db; ++k) dict |= zld8(src + i + k) << (8 * k);
          i += db;
          if (dict) break;
          const uint32_t fb = fcs_flag == 0 ? (single ? 1 : 0) : fcs_flag == 1 ? 2 : fcs_flag == 2 ? 4 : 8;
          if (c.n - i < fb) break;
          uint64_t fcs = 0;
          for (uint32_t k = 0; k < fb; ++k) fcs |= (uint64_t)zld8(src + i + k) << (8 * k);
          if (fb == 2) fcs += 256;
          i += fb;
          if (single) window = fcs;
          if (window > (1ull << 27) + 1) break;
          c.bmax = window < kZBlockMax ? window : kZBlockMax;
          c.fcs = fcs;
          c.fcs_known = fb != 0;
          c.checksum = (fhd >> 2) & 1u;
          c.frame_start = c.o;
          c.have_huf = c.have_ll = c.have_of = c.have_ml = 0;
          c.rep[0] = 1;
          c.rep[1] = 4;
          c.rep[2] = 8;
          c.in_frame = 1;
          c.i = i;
        }
        // block header (3.1.1.2)
        if (c.n - c.i < 3) break;
        const uint32_t bh = zld8(src + c.i) | (zld8(src + c.i + 1) << 8) | (zld8(src + c.i + 2) << 16);
        c.i += 3;
        const uint32_t last = bh & 1u, bt = (bh >> 1) & 3u;
        const uint64_t bs = bh >> 3;
        if (bt == 3 || bs > c.bmax) break;
        c.blk_off = c.i;
        c.blk_len = bs;
        if (bt == 1) {
          if (c.n - c.i < 1 || bs > cap - c.o) break;
          c.i += 1;
          act = kZRle;
        } else {
          if (c.n - c.i < bs) break;
          c.i += bs;
          if (bt == 0) {
            if (bs > cap - c.o) break;
            act = kZRaw;
          } else {
            act = kZComp;
          }
        }
        if (last) c.in_frame = 2;  // the frame ends after this block
        break;
      }
      c.action = act;
      if (act == kZComp) {
        // literals section header (3.1.1.3.1)
        const uint8_t* p = src + c.blk_off;
        const uint64_t n = c.blk_len;
        bool ok = n >= 1;
        const uint32_t b0 = ok ? zld8(p) : 0;
        const uint32_t lt = b0 & 3u, sf = (b0 >> 2) & 3u;
        uint64_t regen = 0, comp = 0, hdr = 0;
        if (ok && lt <= 1) {
          if (sf == 0 || sf == 2) {
            regen = b0 >> 3;
            hdr = 1;
          } else if (sf == 1) {
            ok = n >= 2;
            if (ok) regen = (b0 >> 4) | (zld8(p + 1) << 4);
            hdr = 2;
          } else {
            ok = n >= 3;
            if (ok) regen = (b0 >> 4) | (zld8(p + 1) << 4) | (zld8(p + 2) << 12);
            hdr = 3;
          }
        } else if (ok) {
          hdr = sf <= 1 ? 3 : sf == 2 ? 4 : 5;
          ok = n >= hdr;
          if (ok) {
            uint64_t v = 0;
            for (uint64_t k = 0; k < hdr; ++k) v |= (uint64_t)zld8(p + k) << (8 * k);
            const uint32_t bits = sf <= 1 ? 10 : sf == 2 ? 14 : 18;
            regen = (v >> 4) & ((1u << bits) - 1);
            comp = (v >> (4 + bits)) & ((1u << bits) - 1);
          }
        }
        // every literal of the block is emitted: the block needs regen bytes of room
        ok = ok && regen <= kZBlockMax && regen <= cap - c.o;
        uint64_t q = hdr;
        c.lit_type = lt;
        c.regen = (uint32_t)regen;
        c.huf_new = 0;
        c.n_streams = 0;
        c.err = 0;
        if (ok && lt == 0) {
          ok = n - q >= regen;
          c.lit_src = c.blk_off + q;
          q += regen;
        } else if (ok && lt == 1) {
          ok = n - q >= 1;
          if (ok) c.lit_src = zld8(p + q);
          q += 1;
        } else if (ok) {
          ok = n - q >= comp;
          const uint8_t* cp = p + q;
          uint64_t cl = comp;
          if (ok && lt == 2) {
            uint32_t ns = 0, mb = 0;
            const int64_t t = z_huf_weights(cp, cl, hw, ns, mb, ftab, norm, next);
            ok = t >= 0;
            if (ok) {
              // slots: increasing weight, then symbol; weight k takes 2^(k-1)
              uint32_t rank[kZHufMax + 1] = {0}, pos[kZHufMax + 1];
              for (uint32_t s = 0; s < ns; ++s) rank[hw[s]]++;
              uint32_t start = 0;
              for (uint32_t k = 1; k <= kZHufMax; ++k) {
                pos[k] = start;
                start += rank[k] << (k - 1);
              }
              ok = start == (1u << mb);
              for (uint32_t s = 0; s < ns; ++s) {
                const uint32_t k = hw[s];
                hstart[s] = k ? (uint16_t)pos[k] : 0;
                if (k) pos[k] += 1u << (k - 1);
              }
              c.ns = ns;
              c.huf_bits = mb;
              c.huf_new = 1;
              c.have_huf = ok;
              cp += t;
              cl -= (uint64_t)t;
            }
          } else if (ok && !c.have_huf) {
            ok = false;  // treeless literals without an earlier table
          }
          if (ok && sf == 0) {
            c.n_streams = 1;
            c.seg_off[0] = (uint64_t)(cp - src);
            c.seg_len[0] = cl;
            c.seg_cnt[0] = (uint32_t)regen;
          } else if (ok) {
            ok = regen >= 6 && cl >= 6;
            if (ok) {
              const uint64_t s1 = zld8(cp) | (zld8(cp + 1) << 8), s2 = zld8(cp + 2) | (zld8(cp + 3) << 8),
                             s3 = zld8(cp + 4) | (zld8(cp + 5) << 8);
              const uint64_t seg = (regen + 3) / 4;
              ok = 6 + s1 + s2 + s3 <= cl && regen >= 3 * seg;
              if (ok) {
                c.n_streams = 4;
                const uint64_t b = (uint64_t)(cp - src) + 6;
                c.seg_off[0] = b;
                c.seg_len[0] = s1;
                c.seg_off[1] = b + s1;
                c.seg_len[1] = s2;
                c.seg_off[2] = b + s1 + s2;
                c.seg_len[2] = s3;
                c.seg_off[3] = b + s1 + s2 + s3;
                c.seg_len[3] = cl - 6 - s1 - s2 - s3;
                c.seg_cnt[0] = c.seg_cnt[1] = c.seg_cnt[2] = (uint32_t)seg;
                c.seg_cnt[3] = (uint32_t)(regen - 3 * seg);
              }
            }
          }
          q += comp;
        }
        c.seq_off = c.blk_off + q;
        if (!ok) c.action = kZError;
      }
    }
    __syncthreads();
    const uint32_t act = c.action;
    if (act == kZDone || act == kZError) break;
    if (act == kZRaw) {
      for (uint64_t k = lane; k < c.blk_len; k += 64) z_put(dst, ring, c.o + k, zld8(src + c.blk_off + k));
    } else if (act == kZRle) {
      const uint32_t v = zld8(src + c.blk_off);
      for (uint64_t k = lane; k < c.blk_len; k += 64) z_put(dst, ring, c.o + k, v);
    } else {
      // ---- Huffman literals into the output's last `regen` bytes ----
      if (c.huf_new) {
        const uint32_t mb = c.huf_bits;
        for (uint32_t s = lane; s < c.ns; s += 64) {
          const uint32_t k = hw[s];
          if (!k) continue;
          const uint16_t e = (uint16_t)(s | ((mb + 1 - k) << 8));
          for (uint32_t j = 0, len = 1u << (k - 1); j < len; ++j) huf[hstart[s] + j] = e;
        }
      }
      __syncthreads();
      if (c.n_streams) {
        // Huffman-coded literals: the streams' cache lines touched by the
        // wavefront first (one round of loads), so each lane's word loads,
        // issued a refill ahead, find them in the L2 rather than in HBM.
        // (seg_off / seg_len describe the current block only when it has
        // Huffman streams.)
        const uint64_t a0 = (uint64_t)(src + c.seg_off[0]) & ~63ull;
        const uint64_t a1 = (uint64_t)(src + c.seg_off[c.n_streams - 1] + c.seg_len[c.n_streams - 1]);
        uint32_t sink = 0;
        for (uint64_t a = a0 + 64ull * lane; a < a1; a += 64ull * 64)
          sink += g_ld<uint32_t>(a);
        if (sink == 0xFFFFFFFFu && c.n_streams > 4) c.err = sink;  // never true: keeps the loads
      }
      if (lane < c.n_streams) {
        const uint64_t lit0 = cap - c.regen;
        uint64_t out = lit0;
        for (uint32_t k = 0; k < lane; ++k) out += c.seg_cnt[k];
        ZBits r;
        bool good = zb_init(r, src + c.seg_off[lane], c.seg_len[lane]);
        const uint32_t mb = c.huf_bits;
        for (uint32_t k = 0; good && k < c.seg_cnt[lane]; ++k) {
          const uint32_t e = huf[zb_peek(r, mb)];
          g_st<uint8_t>((uint64_t)(dst + out + k), (uint8_t)e);
          zb_skip(r, e >> 8);
        }
        if (!good || zb_pos(r) != 0) atomicOr(&c.err, 1u);  // each stream consumed exactly
      }
      __syncthreads();
      // ---- sequences (3.1.1.3.2): lane 0 parses the section header and
      // tables, then decodes the sequences kZBatch at a time into LDS; the
      // wavefront executes each batch (literal copies and matches 64 bytes
      // per instruction, history through the LDS ring) ----
      ZBits r;                          // lane 0's reader and FSE states
      uint32_t sl = 0, so = 0, sm = 0;
      if (lane == 0) {
        bool ok = c.err == 0;
        const uint8_t* p = src + c.seq_off;
        const uint64_t n = c.blk_off + c.blk_len - c.seq_off;
        uint64_t q = 0, nseq = 0;
        if (ok) {
          ok = n >= 1;
          if (ok) {
            nseq = zld8(p);
            if (nseq < 128) {
              q = 1;
            } else if (nseq < 255) {
              ok = n >= 2;
              if (ok) nseq = ((nseq - 128) << 8) + zld8(p + 1);
              q = 2;
            } else {
              ok = n >= 3;
              if (ok) nseq = zld8(p + 1) + (zld8(p + 2) << 8) + 0x7F00;
              q = 3;
            }
          }
        }
        if (ok && nseq > 0) {
          ok = n - q >= 1;
          const uint32_t modes = ok ? zld8(p + q) : 0;
          q += 1;
          ok = ok && (modes & 3u) == 0;
          // LL, OF, ML tables (3.1.1.3.2.2): 0 predefined, 1 RLE, 2 described, 3 repeat
          struct T {
            uint32_t* t;
            uint32_t mode, max_sym, max_al, def_n, def_al;
            const int16_t* def;
            uint32_t* have;
          } tabs[3] = {{ll_t, modes >> 6, 35, 9, 36, 6, kLLDef, &c.have_ll},
                       {of_t, (modes >> 4) & 3u, 31, 8, 29, 5, kOFDef, &c.have_of},
                       {ml_t, (modes >> 2) & 3u, 52, 9, 53, 6, kMLDef, &c.have_ml}};
          for (int k = 0; ok && k < 3; ++k) {
            T& x = tabs[k];
            if (x.mode == 0) {
              for (uint32_t s = 0; s < x.def_n; ++s) norm[s] = x.def[s];
              z_fse_build(x.t, norm, x.def_n, x.def_al, next);
              c.al[k] = x.def_al;
              *x.have = 1;
            } else if (x.mode == 1) {
              ok = n - q >= 1 && zld8(p + q) <= x.max_sym;
              if (ok) {
                x.t[0] = zld8(p + q);  // one state, no bits
                c.al[k] = 0;
                *x.have = 1;
              }
              q += 1;
            } else if (x.mode == 2) {
              uint32_t a, ns;
              const int64_t u = z_ncount(p + q, n - q, x.max_al, x.max_sym, norm, a, ns);
              ok = u >= 0;
              if (ok) {
                z_fse_build(x.t, norm, ns, a, next);
                c.al[k] = a;
                *x.have = 1;
                q += (uint64_t)u;
              }
            } else {
              ok = *x.have != 0;
            }
          }
          ok = ok && zb_init(r, p + q, n - q);
          if (ok) {
            sl = zb_read(r, c.al[0]);
            so = zb_read(r, c.al[1]);
            sm = zb_read(r, c.al[2]);
          }
        } else if (ok) {
          ok = q == n;  // no sequences: nothing follows the count
          nseq = 0;
        }
        c.nseq = ok ? nseq : 0;
        c.seq_ok = ok;
        c.seq_wi = r.wi;
        c.seq_base = r.base;
        c.seq_lead = r.lead;
        c.seq_rel = r.rel;
        c.seq_w = r.w;
        c.seq_nx = r.nx;
        c.seq_state[0] = sl;
        c.seq_state[1] = so;
        c.seq_state[2] = sm;
      }
      __syncthreads();
      // every lane runs the sequence chain with wave-uniform values from here
      ZBits q;
      q.base = zu64(c.seq_base);
      q.lead = __builtin_amdgcn_readfirstlane(c.seq_lead);
      q.rel = __builtin_amdgcn_readfirstlane(c.seq_rel);
      q.wi = (int64_t)zu64((uint64_t)c.seq_wi);
      q.w = zu64(c.seq_w);
      q.nx = __builtin_amdgcn_readfirstlane(c.seq_nx);
      uint32_t ql = __builtin_amdgcn_readfirstlane(c.seq_state[0]), qo = __builtin_amdgcn_readfirstlane(c.seq_state[1]),
               qm = __builtin_amdgcn_readfirstlane(c.seq_state[2]);
      const uint64_t regen = __builtin_amdgcn_readfirstlane(c.regen), lit0 = cap - regen, nseq = zu64(c.nseq);
      const uint32_t lt = __builtin_amdgcn_readfirstlane(c.lit_type);
      const uint64_t lit_src = zu64(c.lit_src), frame_start = zu64(c.frame_start);
      auto lit = [&](uint64_t k) -> uint32_t {
        return lt == 0 ? zld8(src + lit_src + k) : lt == 1 ? (uint32_t)(uint8_t)lit_src : zld8(dst + lit0 + k);
      };
      bool ok = c.seq_ok;
      uint64_t o = zu64(c.o), lpos = 0, done = 0;
      while (ok && done < nseq) {
        // the words a batch may read: [wi - kZSeqStage, wi)
        const int64_t stage_lo = c.seq_wi - (int64_t)kZSeqStage;
        for (uint32_t j = lane; j < kZSeqStage; j += 64) {
          const int64_t k = stage_lo + j;
          seq_stage[j] = g_ld<uint32_t>(c.seq_base + 4ull * (uint64_t)(k < 0 ? 0 : k));
        }
        __syncthreads();
        q.sw = (int32_t)kZSeqStage;  // q.wi - stage_lo
        {
          // every lane decodes the batch (the same values in every lane);
          // validation as the serial execution checks it, on copies of the
          // output and literal positions
          // 32-bit positions inside the batch: pb output bytes and lq
          // literals so far (a batch produces under 2^26 bytes); room =
          // cap - o (clamped: the checks below never reach 2^32), lrem =
          // regen - lpos, fs = o - frame_start
          const uint64_t room64 = cap - o, fs = o - frame_start;
          const uint32_t room = room64 > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)room64;
          const uint32_t lrem = (uint32_t)(regen - lpos);
          uint32_t pb = 0, lq = 0, k = 0;
          bool good = true;
          uint32_t rep0 = __builtin_amdgcn_readfirstlane(c.rep[0]), rep1 = __builtin_amdgcn_readfirstlane(c.rep[1]),
                   rep2 = __builtin_amdgcn_readfirstlane(c.rep[2]);
          for (; k < kZBatch && done + k < nseq; ++k) {
            const uint32_t le = __builtin_amdgcn_readfirstlane(ll_t[ql]), oe = __builtin_amdgcn_readfirstlane(of_t[qo]),
                           me = __builtin_amdgcn_readfirstlane(ml_t[qm]);
            const uint32_t ofc = oe & 255u, mlc = me & 255u, llc = le & 255u;
            if (ofc > 31 || mlc > 52 || llc > 35) {
              good = false;
              break;
            }
            const uint32_t mli = __builtin_amdgcn_readlane(ml_code, mlc), lli = __builtin_amdgcn_readlane(ll_code, llc);
            // the window holds >= 32 bits between refills: the offset's
            // extra bits (<= 31), then ML + LL extra bits (<= 16 + 16), then
            // the three state updates (<= 9 + 9 + 8), a refill check after each
            const uint32_t ofv = (1u << ofc) + zs_take(q, ofc);
            zs_fill(q, seq_stage);
            const uint32_t ml = (mli & 0xFFFFFFu) + zs_take(q, mli >> 24);
            const uint32_t ll = (lli & 0xFFFFFFu) + zs_take(q, lli >> 24);
            zs_fill(q, seq_stage);
            uint32_t off;
            if (ofv > 3) {  // 3.1.1.5 repeat offsets
              off = ofv - 3;
              rep2 = rep1;
              rep1 = rep0;
              rep0 = off;
            } else {
              const uint32_t idx = ofv + (ll == 0 ? 1u : 0u);  // 1..4
              if (idx == 1) {
                off = rep0;
              } else {
                off = idx == 2 ? rep1 : idx == 3 ? rep2 : rep0 - 1;
                if (off == 0) {  // idx 4 of rep0 == 1
                  good = false;
                  break;
                }
                if (idx != 2) rep2 = rep1;
                rep1 = rep0;
                rep0 = off;
              }
            }
            if (done + k + 1 < nseq) {
              ql = (le >> 16) + zs_take(q, (le >> 8) & 255u);
              qm = (me >> 16) + zs_take(q, (me >> 8) & 255u);
              qo = (oe >> 16) + zs_take(q, (oe >> 8) & 255u);
              zs_fill(q, seq_stage);
            }
            // execute (3.1.1.4): the writes stay below the unread literals
            // (pb + (lrem - lq) <= room, so the subtraction below stays >= 0)
            if (ll > lrem - lq || pb + (lrem - lq) > room) {
              good = false;
              break;
            }
            pb += ll;
            lq += ll;
            if ((uint64_t)off > fs + pb || ml > room - pb - (lrem - lq)) {
              good = false;
              break;
            }
            if (lane == 0) {
              sq_ll[k] = ll;
              sq_ml[k] = ml;
              sq_off[k] = off;
              sq_src[k] = o + pb - off;
            }
            pb += ml;
          }
          const uint64_t lp = lpos + lq;
          __syncthreads();  // every lane has read c before lane 0 updates it
          if (lane == 0) {
            c.rep[0] = rep0;
            c.rep[1] = rep1;
            c.rep[2] = rep2;
            c.seq_wi = q.wi;
            c.batch = k;
            c.batch_lits = lp - lpos;
            c.seq_ok = good;
          }
        }
        __syncthreads();
        const uint32_t bn = c.batch;
        // the batch's literals (their first kZLitStage bytes) staged in LDS
        // with all their loads issued together
        const uint64_t lit_base = lpos;
        const uint64_t staged = c.batch_lits < kZLitStage ? c.batch_lits : kZLitStage;
        for (uint64_t j0 = 0; j0 < staged; j0 += 16 * 64) {
          uint32_t v[16];
#pragma unroll
          for (uint32_t t = 0; t < 16; ++t) {
            const uint64_t j = j0 + 64 * t + lane;
            v[t] = j < staged ? lit(lit_base + j) : 0u;
          }
#pragma unroll
          for (uint32_t t = 0; t < 16; ++t) {
            const uint64_t j = j0 + 64 * t + lane;
            if (j < staged) lit_stage[j] = (uint8_t)v[t];
          }
        }
        auto blit = [&](uint64_t k) -> uint32_t {  // literal k of the block
          return k - lit_base < staged ? (uint32_t)lit_stage[k - lit_base] : lit(k);
        };
        // the first 8 source bytes of every match reaching past the ring,
        // where they were stored before this batch: eight matches per
        // instruction, all loads issued before the first is used
        const uint64_t ob = o;
        if (o > fence_o) {
          __threadfence_block();
          fence_o = o;
        }
        {
          uint32_t v[kZBatch / 8];
#pragma unroll
          for (uint32_t t = 0; t < kZBatch / 8; ++t) {
            const uint32_t k = 8 * t + lane / 8, j = lane & 7u;
            bool take = false;
            uint64_t a = 0;
            if (k < bn) {
              a = sq_src[k] + j;
              take = sq_off[k] > kZRing && j < sq_ml[k] && a < ob;
            }
            v[t] = take ? zld8(dst + a) : 0u;
          }
#pragma unroll
          for (uint32_t t = 0; t < kZBatch / 8; ++t) sq_pre[8 * (8 * t) + lane] = (uint8_t)v[t];
        }
        for (uint32_t k = 0; k < bn; ++k) {
          const uint32_t ll = sq_ll[k], ml = sq_ml[k], off = sq_off[k];
          for (uint32_t j = lane; j < ll; j += 64) z_put(dst, ring, o + j, blit(lpos + j));
          o += ll;
          lpos += ll;
          // prefetched leading bytes: those below ob, at most 8
          const uint64_t src0 = o - off;
          const uint64_t below = ob > src0 ? ob - src0 : 0;
          const uint32_t pn = off > kZRing ? (uint32_t)(below < 8 ? below : 8) : 0u;
          z_match(dst, ring, o, off, ml, lane, fence_o, sq_pre + 8 * k, pn < ml ? pn : ml);
          o += ml;
        }
        done += bn;
        ok = c.seq_ok;
        __syncthreads();  // lane 0 refills the batch arrays next
      }
      if (lane == 0 && ok && nseq) c.seq_ok = zb_pos(q) == 0;
      __syncthreads();
      ok = ok && c.seq_ok;
      if (ok) {
        for (uint64_t k = lane; k < regen - lpos; k += 64) z_put(dst, ring, o + k, lit(lpos + k));
        o += regen - lpos;
        ok = o - c.o <= c.bmax;
      }
      __syncthreads();  // every lane has read c.o
      if (lane == 0) {
        c.o = o;
        if (!ok) c.action = kZError;
      }
    }
    __syncthreads();
    if (c.action == kZError) break;
    if (lane == 0) {
      if (act != kZComp) c.o += c.blk_len;
      if (c.in_frame == 2) {  // end of frame: content size and checksum
        c.in_frame = 0;
        bool ok = !c.fcs_known || c.o - c.frame_start == c.fcs;
        if (ok && c.checksum) {  // low 32 bits of XXH64 (seed 0) of the frame's content
          ok = c.n - c.i >= 4;
          if (ok) {
            const uint32_t want = zld8(src + c.i) | (zld8(src + c.i + 1) << 8) | (zld8(src + c.i + 2) << 16) |
                                  (zld8(src + c.i + 3) << 24);
            ok = (uint32_t)z_xxh64(dst + c.frame_start, c.o - c.frame_start) == want;
          }
          c.i += 4;
        }
        if (!ok) c.action = kZError;
      }
    }
    __syncthreads();
    if (c.action == kZError) break;
  }
  if (lane == 0) {
    uint32_t st = c.action == kZDone ? kStOk : kStBadStream;
    if (st == kStOk && c.o != cap) st = kStBadLength;
    status[blockIdx.x] = st;
  }
}

hipError_t launch_zstd_decode(const DecodeJob* jobs_dev, uint32_t* status_dev, uint32_t n_jobs, hipStream_t stream) {
  if (n_jobs == 0) return hipSuccess;
  hipLaunchKernelGGL(zstd_decode_kernel, dim3(n_jobs), dim3(64), 0, stream, jobs_dev, status_dev);
  return hipGetLastError();
}

}  // namespace ptwm
