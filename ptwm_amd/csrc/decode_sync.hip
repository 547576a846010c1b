// decode_sync.hip -- parallel decode of the reference's Huffman streams.
//
// A reference Huffman payload has four backward bitstreams
// (entropy/huffman/compress.rs:9-103, bitstream.rs:22-50), each decoded
// serially by the reference (decompress.rs:8-211).  Prefix codes
// resynchronise: a decoder started at an arbitrary bit soon lands on a true
// codeword boundary.  So every stream is cut into subsequences of
// sub_bits bits (480, fewer for launches too small to fill the device), one
// lane each:
//   pass 1   each lane decodes from its subsequence's first bit up to the
//            first codeword boundary at or past its end (its "exit"); lanes
//            of a wavefront then restart from their left neighbour's exit
//            until no start changes; the wavefront publishes its last exit,
//            takes the previous wavefront's (look-back) and restarts its
//            first lane there (sync_pass_kernel; its last workgroups copy
//            stored payloads);
//   fix      the same across wavefronts: a wavefront whose first start
//            differs from the previous wavefront's last exit restarts there
//            (sync_fix_kernel; kFixQueued passes are queued with no host
//            round trip, each skipping its work when the one before changed
//            nothing; a fix of the last of them that moves a wavefront's
//            last exit marks the stream unsettled, and the host queues more
//            passes, checking in between);
//   scan     per stream, symbol counts -> output offsets (sync_scan_kernel);
//   write    each lane decodes its subsequence again and writes the symbols
//            (staged in LDS, stored coalesced) (sync_write_kernel);
//   verdict  the payload is accepted here only when, for all four streams,
//            the end T of symbol n-1 satisfies ceil(T / 8) == stream bytes
//            and the bits after T are zero: the write pass's lane holding
//            symbol n-1 judges its stream (the scan judges a stream without
//            one), and the fourth verdict sets the payload's status.
// Under that condition the reference reader (BitReader, decode_symbol,
// decode_stream_tail) never lets its bit counter wrap and always indexes the
// table with real stream bits, so it produces exactly the zero-padded
// sequential decode and ends exhausted (byte_index < 0, container 0): the
// output here is the reference's, bit for bit.  A payload that fails the
// condition (malformed, or encoded with trailing bytes) is decoded again on
// the exact path, whose state machine replicates the reference for every
// input.
//
// Logical bit k of a stream of m bytes is bit k % 8 of byte m - 1 - k / 8
// (bitstream.rs:58-121); the kernels stage each wavefront's span of the
// stream in LDS in logical order, so a 32-bit window at any bit is two LDS
// words and one funnel shift.
#include "decode_sync.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <vector>

namespace ptwm {

namespace {

constexpr uint32_t kLanes = 64;
// the largest wavefront span, + the window overrun and the bit buffer's look-ahead
constexpr uint32_t kStageWords = kLanes * kSyncSubBitsMax / 32 + 5;
// LDS output staging per wavefront of the write pass: chosen per launch
// from the payloads' expected symbols per wavefront, so that the LDS it
// takes does not cap the occupancy lower than needed (a wavefront with more
// output writes it straight to memory)
constexpr uint32_t kOutStageMax = 16384;
constexpr uint32_t kMaxFixPasses = 256;
static_assert(kSyncSubBitsMax % 64 == 32 && kSyncSubBitsMin % 64 == 32, "subsequence sizes: odd word counts");

// Which stream of deferred payload d, and which wavefront of it, wavefront
// `w` of the payload's launch range covers; -1 when past the last.
__device__ inline int locate(const SyncStream* S4, uint32_t& w) {
  for (int s = 0; s < 4; ++s) {
    const uint32_t ws = (S4[s].n_sub + kLanes - 1) / kLanes;
    if (w < ws) return s;
    w -= ws;
  }
  return -1;
}

__device__ inline uint8_t gbyte(uint64_t a) {
  return *(const __attribute__((address_space(1))) uint8_t*)(uintptr_t)a;
}

// Stage logical bytes [L0, L0 + 4 (2 sub_bits + 5)) of the stream in LDS
// (a wavefront's span and the look-ahead; logical order, zero past the
// stream's end) and its decode table.
__device__ inline void stage_wave(const SyncStream& S, uint64_t L0, const uint16_t* __restrict__ tables,
                                  uint32_t* stage, uint16_t* tab) {
  const uint32_t lane = threadIdx.x;
  const uint32_t tsize = 1u << S.max_bits;  // >= 2
  // Every load is issued before the first LDS store, none of them under a
  // condition, so the wavefront waits for memory once.  The table: the
  // payload's whole slot (2048 entries, 4 KiB) in 16-byte loads.
  constexpr uint32_t kTabIt = kSyncTableEntries / (8 * kLanes);
  const uint64_t gt = reinterpret_cast<uint64_t>(tables + (uint64_t)kSyncTableEntries * S.table);
  u32x4 t4[kTabIt];
#pragma unroll
  for (uint32_t it = 0; it < kTabIt; ++it) t4[it] = g_ld<u32x4>(gt + 16ull * (lane + kLanes * it));
  // Logical bytes [b, b + 4) of a stage word are the physical bytes
  // [m - 4 - b, m - 1 - b] reversed: one byte swap of the word at a =
  // src + m - 4 - b, read as the aligned words that hold it.  Bytes past the
  // stream's logical end are masked to zero; the address of a word wholly
  // past it is clamped to src - 8, which still lies in the payload (ahead
  // of the streams sit the tag, the weights header and the jump table).
  constexpr uint32_t kStIt = (kStageWords + kLanes - 1) / kLanes;
  // (words past the span are loaded too, at in-bounds addresses, and not
  // stored: a load under a condition would make the stores wait for each)
  const uint32_t n_words = 2 * S.sub_bits + 5;
  const uint64_t lo_min = (S.src - 8) & ~3ull;
  uint32_t w0[kStIt], w1[kStIt];
#pragma unroll
  for (uint32_t it = 0; it < kStIt; ++it) {
    const uint64_t b = L0 + 4ull * (lane + kLanes * it);
    const uint64_t a = S.src + S.m - 4 - b;
    const uint64_t lo = std::max<uint64_t>(a & ~3ull, lo_min);
    w0[it] = g_ld<uint32_t>(lo);
    w1[it] = g_ld<uint32_t>((a & 3u) ? lo + 4 : lo);
  }
  // (tsize >= 2: a table is stored as whole 32-bit words)
  uint32_t* const t32 = reinterpret_cast<uint32_t*>(tab);
#pragma unroll
  for (uint32_t it = 0; it < kTabIt; ++it) {
    const uint32_t i = 4 * (lane + kLanes * it);
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k)
      if (2 * (i + k) < tsize) t32[i + k] = t4[it][k];
  }
#pragma unroll
  for (uint32_t it = 0; it < kStIt; ++it) {
    const uint32_t q = lane + kLanes * it;
    const uint64_t b = L0 + 4ull * q;
    const uint64_t a = S.src + S.m - 4 - b;
    const uint64_t rem = b < S.m ? S.m - b : 0;
    const uint32_t keep = rem >= 4 ? 0xFFFFFFFFu : (uint32_t)((1ull << (8 * rem)) - 1ull);
    const uint32_t v = __builtin_bswap32(__builtin_amdgcn_alignbyte(w1[it], w0[it], (uint32_t)(a & 3u))) & keep;
    if (q < n_words) stage[q] = v;
  }
  __syncthreads();
}

// A bit reader over the staged span: 64 bits from position p in a register
// pair (at least 32 valid at the top of each step) and the stage word that
// follows them, loaded at the previous refill.  A step takes at most 22 bits
// (two codewords); a refill shifts that word in and loads the next one, so
// the word a refill consumes has been in flight for at least one step (its
// LDS latency overlaps the table lookups) and the load lands in the
// register it is consumed from.
struct Cursor {
  uint64_t buf;
  uint32_t nb, nxt, nidx, p;
};
__device__ inline Cursor cur_open(const uint32_t* stage, uint32_t p) {
  const uint32_t i = p >> 5, sh = p & 31u;
  Cursor c;
  c.buf = ((((uint64_t)stage[i + 1]) << 32) | stage[i]) >> sh;
  c.nb = 64 - sh;
  c.nxt = stage[i + 2];
  c.nidx = i + 3;
  c.p = p;
  return c;
}
__device__ inline uint32_t cur_win(const Cursor& c) { return (uint32_t)c.buf; }
__device__ inline void cur_adv(Cursor& c, const uint32_t* stage, uint32_t n) {
  c.buf >>= n;
  c.nb -= n;
  c.p += n;
  if (c.nb < 32) {
    c.buf |= (uint64_t)c.nxt << c.nb;
    c.nb += 32;
    c.nxt = stage[c.nidx++];
  }
}

// Decode from bit p (relative to the staged span) until p >= stop; returns
// the exit bit, symbol count in `cnt`.  Every codeword is >= 1 bit; two per
// window (the second from the window's bits after the first: 32 - 11 >= 11).
__device__ inline uint32_t run(const uint32_t* stage, const uint16_t* tab, uint32_t mask, uint32_t p, uint32_t stop,
                               uint32_t& cnt) {
  uint32_t c = 0;
  Cursor k = cur_open(stage, p);
  while (k.p < stop) {
    const uint32_t win = cur_win(k);
    const uint32_t l1 = tab[win & mask] >> 8;
    const uint32_t l2 = tab[(win >> l1) & mask] >> 8;  // looked up whether or not it is taken
    const bool two = k.p + l1 < stop;
    cur_adv(k, stage, two ? l1 + l2 : l1);
    c += two ? 2u : 1u;
  }
  cnt = c;
  return k.p;
}

// Codeword starts of a lane's path, one bit per bit of its subsequence:
// word w of lane l at bm[w * kLanes + l] (consecutive lanes, consecutive banks).
constexpr uint32_t kSubWordsMax = kSyncSubBitsMax / 32;

// run() that also records the path's codeword starts (relative to base, the
// lane's subsequence start) in the lane's bitmap.  A codeword is at most
// kHufMaxBits < 32 bits, so consecutive starts never skip a bitmap word.
__device__ inline uint32_t run_rec(const uint32_t* stage, const uint16_t* tab, uint32_t mask, uint32_t base,
                                   uint32_t p, uint32_t stop, uint32_t& cnt, uint32_t* bm) {
  const uint32_t lane = threadIdx.x, sw = (stop - base) >> 5;
  uint32_t c = 0, wi = (p - base) >> 5, bits = 0;
  for (uint32_t w = 0; w < wi; ++w) bm[w * kLanes + lane] = 0u;
  Cursor k = cur_open(stage, p);
  while (k.p < stop) {
    const uint32_t p0 = k.p;
    const uint32_t win = cur_win(k);
    const uint32_t l1 = tab[win & mask] >> 8;
    const uint32_t l2 = tab[(win >> l1) & mask] >> 8;  // looked up whether or not it is taken
    const bool two = p0 + l1 < stop;
    cur_adv(k, stage, two ? l1 + l2 : l1);
    c += two ? 2u : 1u;
    // record the starts after the step, so that no lookup waits for a bitmap store
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if (j && !two) break;
      const uint32_t rel = (j ? p0 + l1 : p0) - base, w = rel >> 5;
      if (w != wi) {
        bm[wi * kLanes + lane] = bits;
        wi = w;
        bits = 0;
      }
      bits |= 1u << (rel & 31u);
    }
  }
  bm[wi * kLanes + lane] = bits;
  for (uint32_t w = wi + 1; w < sw; ++w) bm[w * kLanes + lane] = 0u;
  cnt = c;
  return k.p;
}

// Restart a lane whose bitmap holds its current path from a new start p:
// decode until a position of the old path (its continuation, and so the
// exit, is the old one: the count is the new prefix plus the old path's
// starts from there), or, without meeting it, to the end; updates ex / cnt.
__device__ inline void run_join(const uint32_t* stage, const uint16_t* tab, uint32_t mask, uint32_t base,
                                uint32_t p, uint32_t stop, uint32_t& ex, uint32_t& cnt, const uint32_t* bm) {
  const uint32_t lane = threadIdx.x, sw = (stop - base) >> 5;
  uint32_t c = 0, wi = (p - base) >> 5, cur = bm[wi * kLanes + lane];
  Cursor k = cur_open(stage, p);
  while (k.p < stop) {
    const uint32_t rel = k.p - base, w = rel >> 5;
    if (w != wi) {
      wi = w;
      cur = bm[wi * kLanes + lane];
    }
    if ((cur >> (rel & 31u)) & 1u) {
      uint32_t rest = __popc(cur >> (rel & 31u));
      for (uint32_t v = wi + 1; v < sw; ++v) rest += __popc(bm[v * kLanes + lane]);
      cnt = c + rest;
      return;  // ex unchanged
    }
    cur_adv(k, stage, tab[cur_win(k) & mask] >> 8);
    ++c;
  }
  ex = k.p;
  cnt = c;
}

// Lanes restart from their left neighbour's exit until no start changes (at
// most 63 rounds: each round fixes at least one more lane).  With a bitmap
// (bm non-null; bm_ok: it holds the lane's current path, updated here) a
// restart stops where it joins the old path; a lane's later restarts run in
// full and record again.
__device__ inline void settle(const uint32_t* stage, const uint16_t* tab, uint32_t mask, uint32_t sb, bool valid,
                              uint32_t& st, uint32_t& ex, uint32_t& cnt, bool& changed, uint32_t* bm, bool& bm_ok) {
  const uint32_t lane = threadIdx.x;
  const uint32_t base = lane * sb, stop = base + sb;
  for (uint32_t round = 0; round < kLanes; ++round) {
    const uint32_t prev = (uint32_t)__shfl_up((int)ex, 1, 64);
    const bool ch = valid && lane > 0 && prev != st;
    if (__ballot(ch) == 0) break;
    if (ch) {
      st = prev;
      if (bm && bm_ok) {
        run_join(stage, tab, mask, base, st, stop, ex, cnt, bm);
        bm_ok = false;  // the bitmap now also holds starts of the replaced prefix
      } else if (bm) {
        ex = run_rec(stage, tab, mask, base, st, stop, cnt, bm);
        bm_ok = true;
      } else {
        ex = run(stage, tab, mask, st, stop, cnt);
      }
      changed = true;
    }
  }
}
__device__ inline void settle(const uint32_t* stage, const uint16_t* tab, uint32_t mask, uint32_t sb, bool valid,
                              uint32_t& st, uint32_t& ex, uint32_t& cnt, bool& changed) {
  bool no_bm = false;
  settle(stage, tab, mask, sb, valid, st, ex, cnt, changed, nullptr, no_bm);
}

// Stored bytes the exact kernel deferred (copy_src[j] != 0): output bytes
// [a, b) of job J, by nt threads.  Aligned dword stores; the source is
// realigned with a funnel shift of two aligned words, used only where both
// words hold source bytes.
__device__ inline void copy_range(const DecodeJob& J, uint64_t s, uint64_t a, uint64_t b, uint32_t t, uint32_t nt) {
  const uint64_t ba = J.dst + a, bb = J.dst + b;
  const uint64_t lo = std::min<uint64_t>((ba + 3) & ~3ull, bb);
  const uint64_t hi = std::max<uint64_t>(bb & ~3ull, lo);
  for (uint64_t x = ba + t; x < lo; x += nt) g_st<uint8_t>(x, g_ld<uint8_t>(s + (x - J.dst)));
  for (uint64_t x = hi + t; x < bb; x += nt) g_st<uint8_t>(x, g_ld<uint8_t>(s + (x - J.dst)));
#pragma unroll 4
  for (uint64_t x = lo + 4ull * t; x < hi; x += 4ull * nt) {
    const uint64_t o = x - J.dst;
    if (o + 5 <= J.dst_len) {
      const uint64_t S = s + o;
      const uint64_t sa = S & ~3ull;
      g_st<uint32_t>(x, __builtin_amdgcn_alignbyte(g_ld<uint32_t>(sa + 4), g_ld<uint32_t>(sa), (uint32_t)(S & 3u)));
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) g_st<uint8_t>(x + k, g_ld<uint8_t>(s + o + k));
    }
  }
}

// Deferred stored-bytes copies as workgroups of `parts` pieces per
// copy_chunk(len) of output: piece i of the launch's copy range.
struct CopyArgs {
  const DecodeJob* jobs;
  const uint64_t* copy_src;
  const uint32_t* chunk_job;
  const uint32_t* job_chunk0;
};
__device__ inline void copy_piece(const CopyArgs& C, uint32_t i, uint32_t parts, uint32_t t, uint32_t nt) {
  const uint32_t c = i / parts, q = i % parts;
  const uint32_t j = C.chunk_job[c];
  const uint64_t s = C.copy_src[j];
  if (s == 0) return;
  const DecodeJob J = C.jobs[j];
  const uint64_t cs = copy_chunk(J.dst_len), ps = cs / parts;
  const uint64_t a = (uint64_t)(c - C.job_chunk0[j]) * cs + q * ps;
  const uint64_t b = std::min<uint64_t>(J.dst_len, a + ps);
  if (a < b) copy_range(J, s, a, b, t, nt);
}

__global__ void __launch_bounds__(256) raw_copy_kernel(CopyArgs C) { copy_piece(C, blockIdx.x, 1, threadIdx.x, 256); }

__device__ inline uint32_t wave_total(uint32_t c) {
  for (int o = 32; o >= 1; o >>= 1) c += (uint32_t)__shfl_xor((int)c, o, 64);
  return c;
}

// The previous wavefront of the stream publishes where its last lane's path
// leaves its span: pub[wavefront] = (epoch << 8) | (exit - span end), the
// overrun of a codeword (< kHufMaxBits bits).  A reader waits for it at most
// kLookBackTicks of the 100 MHz clock; without it the fix pass does the work.
constexpr uint64_t kLookBackTicks = 2000;
__device__ inline bool look_back(const uint64_t* pub, uint32_t wave, uint64_t epoch, uint32_t& rel) {
  const uint64_t t_end = __builtin_amdgcn_s_memrealtime() + kLookBackTicks;
  for (;;) {
    const uint64_t v = __hip_atomic_load(pub + wave, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    const uint64_t u = ((uint64_t)hi << 32) | lo;
    if ((u >> 8) == epoch) {
      rel = (uint32_t)(u & 0xFFu);
      return true;
    }
    if (__builtin_amdgcn_s_memrealtime() > t_end) return false;
    __builtin_amdgcn_s_sleep(4);
  }
}

// First pass.  Each lane decodes its subsequence, recording its codeword
// starts; the lanes settle; the wavefront publishes its last exit, takes
// the previous wavefront's (look-back), restarts its first lane there (a
// join on the recorded path) and settles again.  Workgroups past the
// wavefronts copy deferred stored bytes (four per copy piece).
__global__ void __launch_bounds__(64) sync_pass_kernel(const SyncStream* __restrict__ streams,
                                                       const uint32_t* __restrict__ wave_job,
                                                       const uint32_t* __restrict__ job_wave0,
                                                       const uint16_t* __restrict__ tables, SyncArrays A,
                                                       uint32_t nw, CopyArgs C) {
  __shared__ uint16_t tab[kSyncTableEntries];
  __shared__ uint32_t stage[kStageWords];
  __shared__ uint32_t bm[kSubWordsMax * kLanes];
  if (blockIdx.x >= nw) {
    copy_piece(C, blockIdx.x - nw, 4, threadIdx.x, kLanes);
    return;
  }
  const uint32_t d = wave_job[blockIdx.x];
  uint32_t w = blockIdx.x - job_wave0[d];
  const int s = locate(streams + 4ull * d, w);
  if (s < 0) return;
  const SyncStream S = streams[4ull * d + s];
  const uint32_t sb = S.sub_bits;
  const uint64_t L0 = (uint64_t)w * kLanes * (sb / 8);
  const uint32_t lane = threadIdx.x, k = w * kLanes + lane;
  const bool valid = k < S.n_sub;
  const uint64_t g = (uint64_t)S.first_sub + k;
  if (S.fixed_len) {
    // a fixed-length code: codeword starts are the multiples of its length,
    // so each lane's start, count and exit are arithmetic (and the wavefronts
    // agree with their neighbours: nothing to settle)
    const uint32_t L = S.fixed_len;
    uint32_t n = 0;
    if (valid) {
      const uint64_t a0 = L0 * 8 + (uint64_t)lane * sb;
      const uint64_t stop = a0 + sb;
      const uint64_t st = (a0 + L - 1) / L * L;
      n = st < stop ? (uint32_t)((stop - st + L - 1) / L) : 0u;
      A.start[g] = st;
      A.exit[g] = st + (uint64_t)n * L;
      A.count[g] = n;
    }
    const uint32_t tot = wave_total(n);
    if (lane == 0) A.wave_sum[blockIdx.x] = tot;
    return;
  }
  stage_wave(S, L0, tables, stage, tab);
  const uint32_t mask = (1u << S.max_bits) - 1;
  uint32_t st = lane * sb, cnt = 0, ex = st;
  if (valid) ex = run_rec(stage, tab, mask, st, st, st + sb, cnt, bm);
  bool changed = false, bm_ok = valid;
  settle(stage, tab, mask, sb, valid, st, ex, cnt, changed, bm, bm_ok);
  if (lane == kLanes - 1 && valid && k + 1 < S.n_sub)
    __hip_atomic_store(A.pub + blockIdx.x, (A.epoch << 8) | (uint64_t)(ex - kLanes * sb), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  uint32_t rel = 0;
  if (w > 0 && A.look_back && look_back(A.pub, blockIdx.x - 1, A.epoch, rel) && rel != 0 && rel < sb) {
    // the true first start lies rel bits into the span: lane 0 joins its
    // recorded path from there (it never restarted, so the bitmap is its
    // path), and a changed exit propagates as in the first settle
    if (lane == 0) {
      st = rel;
      run_join(stage, tab, mask, 0, st, sb, ex, cnt, bm);
      bm_ok = false;
    }
    settle(stage, tab, mask, sb, valid, st, ex, cnt, changed, bm, bm_ok);
  }
  if (valid) {
    A.start[g] = L0 * 8 + st;
    A.exit[g] = L0 * 8 + ex;
    A.count[g] = cnt;
  }
  const uint32_t tot = wave_total(valid ? cnt : 0u);
  if (lane == 0) A.wave_sum[blockIdx.x] = tot;
}

// Fix passes: a wavefront whose first start differs from the previous
// wavefront's last exit restarts from it and settles again.  A workgroup
// checks 64 wavefronts at once (a lane each) and fixes those that need it.
// With mark 1 (the last pass queued without a host check), a fix that moves
// a wavefront's last exit marks the stream unsettled: the next wavefront
// may have been checked against the old exit.  With mark 2 any fix does (a
// test mode that drives the host's extra passes).
__device__ inline void fix_wave(SyncStream* __restrict__ streams, const uint32_t* __restrict__ wave_job,
                                const uint32_t* __restrict__ job_wave0, const uint16_t* __restrict__ tables,
                                const SyncArrays& A, uint32_t wl, uint32_t mark, uint32_t* tab32, uint32_t* stage) {
  uint16_t* const tab = reinterpret_cast<uint16_t*>(tab32);
  const uint32_t d = wave_job[wl];
  uint32_t w = wl - job_wave0[d];
  const int s = locate(streams + 4ull * d, w);
  const SyncStream S = streams[4ull * d + s];
  const uint64_t g0 = (uint64_t)S.first_sub + (uint64_t)w * kLanes;
  const uint64_t prev_exit = A.exit[g0 - 1];
  const uint32_t sb = S.sub_bits;
  const uint64_t L0 = (uint64_t)w * kLanes * (sb / 8);
  __syncthreads();  // the previous wavefront's reads of the staged span are done
  stage_wave(S, L0, tables, stage, tab);
  const uint32_t lane = threadIdx.x, mask = (1u << S.max_bits) - 1;
  const uint32_t k = w * kLanes + lane;
  const bool valid = k < S.n_sub;
  uint32_t st = 0, ex = 0, cnt = 0;
  if (valid) {
    st = (uint32_t)(A.start[g0 + lane] - L0 * 8);
    ex = (uint32_t)(A.exit[g0 + lane] - L0 * 8);
    cnt = A.count[g0 + lane];
  }
  const uint32_t ex_before = ex;
  bool changed = false;
  if (lane == 0) {  // prev_exit lies in [L0 * 8, L0 * 8 + 11): a codeword overruns by < 11 bits
    st = (uint32_t)std::min<uint64_t>(prev_exit - L0 * 8, sb);
    ex = run(stage, tab, mask, st, sb, cnt);
    changed = true;
  }
  settle(stage, tab, mask, sb, valid, st, ex, cnt, changed);
  if (valid && changed) {
    A.start[g0 + lane] = L0 * 8 + st;
    A.exit[g0 + lane] = L0 * 8 + ex;
    A.count[g0 + lane] = cnt;
  }
  const uint32_t tot = wave_total(valid ? cnt : 0u);
  if (lane == 0) A.wave_sum[wl] = tot;
  if (mark && lane == kLanes - 1 && ((valid && k + 1 < S.n_sub && ex != ex_before) || mark == 2))
    streams[4ull * d + s].pad = 1u;
}

__global__ void __launch_bounds__(64) sync_fix_kernel(SyncStream* __restrict__ streams,
                                                      const uint32_t* __restrict__ wave_job,
                                                      const uint32_t* __restrict__ job_wave0,
                                                      const uint16_t* __restrict__ tables, SyncArrays A, uint32_t nw,
                                                      const uint32_t* __restrict__ prev_flag,
                                                      uint32_t* __restrict__ flag, uint32_t mark) {
  __shared__ uint32_t tab32[kSyncTableEntries / 2];
  __shared__ uint32_t stage[kStageWords];
  // the previous pass (queued before this one) changed nothing: settled
  if (prev_flag && g_ld<uint32_t>(reinterpret_cast<uint64_t>(prev_flag)) == 0) return;
  const uint32_t lane = threadIdx.x;
  bool any = false;
  for (uint32_t c = blockIdx.x * kLanes; c < nw; c += gridDim.x * kLanes) {
    const uint32_t wl = c + lane;
    bool need = false;
    if (wl < nw) {
      const uint32_t d = wave_job[wl];
      uint32_t w = wl - job_wave0[d];
      const int s = locate(streams + 4ull * d, w);
      if (s >= 0 && w > 0) {
        const uint64_t g0 = (uint64_t)streams[4ull * d + s].first_sub + (uint64_t)w * kLanes;
        need = A.exit[g0 - 1] != A.start[g0];
      }
    }
    uint64_t m = __ballot(need);
    any |= m != 0;
    while (m) {
      const uint32_t i = (uint32_t)__builtin_ctzll(m);
      m &= m - 1;
      fix_wave(streams, wave_job, job_wave0, tables, A, c + i, mark, tab32, stage);
    }
  }
  if (any && lane == 0) *flag = 1u;
}

// A stream's verdict under the exactness condition, reported once per
// stream into its payload's word (bit s: reported, 4 + s: failed, 8 + s:
// unsettled); the report that completes the four sets the payload's status,
// unless the exact kernel gave it a final one (a rejected header: the
// stream records keep the host's zeros, max_bits 0).
__device__ inline void report_stream(const SyncStream& S, uint32_t s, uint32_t* verdict, uint32_t d, bool ok,
                                     uint32_t* status) {
  const uint32_t mine = (1u << s) | (ok ? 0u : 1u << (4 + s)) | (S.pad ? 1u << (8 + s) : 0u);
  const uint32_t all = atomicOr(verdict + d, mine) | mine;
  if ((all & 0xFu) != 0xFu || ((all ^ mine) & 0xFu) == 0xFu) return;
  if (S.max_bits == 0) return;
  status[S.job] = (all & 0xF00u) ? kStUnsettled : (all & 0xF0u) ? kStFallback : kStOk;
}

// The condition for a stream whose symbol n-1 ends at bit T.
__device__ inline bool stream_exact(const SyncStream& S, uint64_t T) {
  if (T > 8 * S.m || T <= 8 * (S.m - 1)) return false;
  const uint32_t used = (uint32_t)(T - 8 * (S.m - 1));  // bits of the last logical byte, 1..8
  return used == 8 || (gbyte(S.src) >> used) == 0;
}

// Exclusive scan of the wavefront sums of one stream (blockIdx.x = 4 d + s);
// its wavefronts are consecutive in the launch, after those of streams < s.
__global__ void __launch_bounds__(256) sync_scan_kernel(const SyncStream* __restrict__ streams,
                                                        const uint32_t* __restrict__ job_wave0, SyncArrays A,
                                                        uint32_t* __restrict__ status) {
  __shared__ uint64_t part[256];
  const uint32_t d = blockIdx.x / 4, s = blockIdx.x % 4;
  uint32_t w0 = job_wave0[d];
  for (uint32_t i = 0; i < s; ++i) w0 += (streams[4ull * d + i].n_sub + kLanes - 1) / kLanes;
  const uint32_t nw = (streams[blockIdx.x].n_sub + kLanes - 1) / kLanes;
  const uint32_t t = threadIdx.x;
  const uint32_t per = (nw + 255) / 256;
  const uint32_t a = std::min(nw, t * per), b = std::min(nw, a + per);
  uint64_t sum = 0;
  for (uint32_t k = a; k < b; ++k) sum += A.wave_sum[w0 + k];
  part[t] = sum;
  __syncthreads();
  for (uint32_t o = 1; o < 256; o <<= 1) {  // inclusive Hillis-Steele scan
    const uint64_t v = t >= o ? part[t - o] : 0;
    __syncthreads();
    part[t] += v;
    __syncthreads();
  }
  uint64_t acc = t ? part[t - 1] : 0;
  for (uint32_t k = a; k < b; ++k) {
    A.wave_prefix[w0 + k] = acc;
    acc += A.wave_sum[w0 + k];
  }
  // a stream with no symbol n-1 (none expected, or too few decoded) is
  // judged here; every other stream by the write pass's wavefront holding it
  const SyncStream& S = streams[blockIdx.x];
  if (t == 0 && (S.n == 0 || part[255] < S.n))
    report_stream(S, s, A.verdict, d, S.n == 0 && S.m == 0, status);
}

// Symbols [0, m) of a lane of a fixed-length code (length L, K L <= 32)
// from bit p0: K independent lookups per window of the bit reader, into the
// LDS output staging (o) or straight to memory (gd).
template <uint32_t K, bool kStaged>
__device__ inline void write_fixed(const uint32_t* stage, const uint16_t* tab, uint32_t mask, uint32_t L, uint32_t p0,
                                   uint32_t m, uint8_t* o, uint64_t gd) {
  Cursor k = cur_open(stage, p0);
  uint32_t i = 0;
  for (; i + K <= m; i += K) {
    const uint32_t win = cur_win(k);
    uint32_t e[K];
#pragma unroll
    for (uint32_t j = 0; j < K; ++j) e[j] = tab[(win >> (j * L)) & mask];
    cur_adv(k, stage, K * L);
#pragma unroll
    for (uint32_t j = 0; j < K; ++j) {
      if constexpr (kStaged) o[i + j] = (uint8_t)e[j];
      else g_st<uint8_t>(gd + i + j, (uint8_t)e[j]);
    }
  }
  for (; i < m; ++i) {
    const uint32_t e = tab[cur_win(k) & mask];
    cur_adv(k, stage, L);
    if constexpr (kStaged) o[i] = (uint8_t)e;
    else g_st<uint8_t>(gd + i, (uint8_t)e);
  }
}
template <bool kStaged>
__device__ inline void write_fixed_any(const uint32_t* stage, const uint16_t* tab, uint32_t mask, uint32_t L,
                                       uint32_t p0, uint32_t m, uint8_t* o, uint64_t gd) {
  if (L <= 4) write_fixed<8, kStaged>(stage, tab, mask, L, p0, m, o, gd);
  else if (L <= 8) write_fixed<4, kStaged>(stage, tab, mask, L, p0, m, o, gd);
  else if (L <= 10) write_fixed<3, kStaged>(stage, tab, mask, L, p0, m, o, gd);
  else write_fixed<2, kStaged>(stage, tab, mask, L, p0, m, o, gd);
}

// Decode again from the settled starts and write symbols [0, n) of the
// segment; the lane holding symbol n-1 records where it ends.  Symbols are
// staged in LDS at their output address mod 16, so the store is dwordx4.
template <uint32_t kOutStage>
__global__ void __launch_bounds__(64) sync_write_kernel(const SyncStream* __restrict__ streams,
                                                        const uint32_t* __restrict__ wave_job,
                                                        const uint32_t* __restrict__ job_wave0,
                                                        const uint16_t* __restrict__ tables, SyncArrays A,
                                                        uint32_t* __restrict__ status) {
  __shared__ uint16_t tab[kSyncTableEntries];
  __shared__ uint32_t stage[kStageWords];
  __shared__ __attribute__((aligned(16))) uint8_t out[kOutStage + 16];
  const uint32_t d = wave_job[blockIdx.x];
  uint32_t w = blockIdx.x - job_wave0[d];
  const int s = locate(streams + 4ull * d, w);
  if (s < 0) return;
  const SyncStream S = streams[4ull * d + s];
  const uint64_t base = A.wave_prefix[blockIdx.x];
  if (base >= S.n) return;  // the whole wavefront decodes padding
  const uint64_t L0 = (uint64_t)w * kLanes * (S.sub_bits / 8);
  stage_wave(S, L0, tables, stage, tab);
  const uint32_t lane = threadIdx.x, mask = (1u << S.max_bits) - 1;
  const uint64_t g = (uint64_t)S.first_sub + (uint64_t)w * kLanes + lane;
  const bool valid = w * kLanes + lane < S.n_sub;
  const uint32_t cnt = valid ? A.count[g] : 0u;
  uint32_t incl = cnt;  // in-wave inclusive scan of the counts
  for (uint32_t o = 1; o < kLanes; o <<= 1) {
    const uint32_t v = (uint32_t)__shfl_up((int)incl, o, 64);
    if (lane >= o) incl += v;
  }
  const uint64_t first = base + (incl - cnt);
  const uint64_t wave_end = std::min<uint64_t>(S.n, base + A.wave_sum[blockIdx.x]);
  const uint64_t wave_len = wave_end - base;
  const bool staged = wave_len <= kOutStage;
  const uint64_t gA = S.dst + base, gB = S.dst + wave_end;
  const uint32_t skew = (uint32_t)(gA & 15u);
  if (valid && first < S.n && S.fixed_len) {
    // fixed-length code: symbol i starts at start + i L, so the lookups do
    // not depend on each other
    const uint32_t L = S.fixed_len, p0 = (uint32_t)(A.start[g] - L0 * 8);
    const uint32_t m = (uint32_t)std::min<uint64_t>(cnt, S.n - first);
    uint8_t* const o = out + skew + (first - base);
    const uint64_t gd = S.dst + first;
    if (staged) write_fixed_any<true>(stage, tab, mask, L, p0, m, o, gd);
    else write_fixed_any<false>(stage, tab, mask, L, p0, m, o, gd);
    if (first + m == S.n) report_stream(S, (uint32_t)s, A.verdict, d, stream_exact(S, L0 * 8 + p0 + m * L), status);
  } else if (valid && first < S.n) {
    Cursor k = cur_open(stage, (uint32_t)(A.start[g] - L0 * 8));
    const uint32_t m = (uint32_t)std::min<uint64_t>(cnt, S.n - first);
    // pairs of symbols with no branch inside the loop (the reader advanced
    // before the stores, so no step waits for its own stores), the odd last
    // symbol after it; staged or not is the same for the whole wavefront
    uint32_t i = 0;
    if (staged) {
      uint8_t* const o = out + skew + (first - base);
      for (; i + 2 <= m; i += 2) {
        const uint32_t win = cur_win(k);
        const uint32_t e1 = tab[win & mask], l1 = e1 >> 8;
        const uint32_t e2 = tab[(win >> l1) & mask];
        cur_adv(k, stage, l1 + (e2 >> 8));
        o[i] = (uint8_t)e1;
        o[i + 1] = (uint8_t)e2;
      }
      if (i < m) {
        const uint32_t e1 = tab[cur_win(k) & mask];
        cur_adv(k, stage, e1 >> 8);
        o[i] = (uint8_t)e1;
      }
    } else {
      for (; i + 2 <= m; i += 2) {
        const uint32_t win = cur_win(k);
        const uint32_t e1 = tab[win & mask], l1 = e1 >> 8;
        const uint32_t e2 = tab[(win >> l1) & mask];
        cur_adv(k, stage, l1 + (e2 >> 8));
        g_st<uint8_t>(S.dst + first + i, (uint8_t)e1);
        g_st<uint8_t>(S.dst + first + i + 1, (uint8_t)e2);
      }
      if (i < m) {
        const uint32_t e1 = tab[cur_win(k) & mask];
        cur_adv(k, stage, e1 >> 8);
        g_st<uint8_t>(S.dst + first + i, (uint8_t)e1);
      }
    }
    if (first + m == S.n) report_stream(S, (uint32_t)s, A.verdict, d, stream_exact(S, L0 * 8 + k.p), status);
  }
  if (staged) {
    __syncthreads();
    const uint64_t al0 = std::min<uint64_t>((gA + 15) & ~15ull, gB);
    const uint64_t al1 = std::max<uint64_t>(gB & ~15ull, al0);
    const uint64_t lbase = gA & ~15ull;  // LDS offset of address X is X - lbase
    for (uint64_t x = gA + lane; x < al0; x += kLanes) g_st<uint8_t>(x, out[x - lbase]);
    for (uint64_t x = al1 + lane; x < gB; x += kLanes) g_st<uint8_t>(x, out[x - lbase]);
    for (uint64_t x = al0 + 16ull * lane; x < al1; x += 16ull * kLanes)
      g_st<u32x4>(x, *reinterpret_cast<const u32x4*>(out + (x - lbase)));
  }
}

}  // namespace

namespace {

#define PTWM_HIP_TRY_ERR(expr)          \
  do {                                  \
    const hipError_t _e = (expr);       \
    if (_e != hipSuccess) return _e;    \
  } while (0)

// Before the offsets and the write are run again: the streams' unsettled
// marks and the payloads' verdict words cleared.
__global__ void __launch_bounds__(256) clear_unsettled_kernel(SyncStream* __restrict__ streams, uint32_t* verdict,
                                                              uint32_t n_def) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i < 4 * n_def) streams[i].pad = 0u;
  if (i < n_def) verdict[i] = 0u;
}

// Per-stream offsets and the write; the streams' verdicts set the deferred
// payloads' statuses (after the fix passes).
hipError_t sync_finish(hipStream_t s, SyncStream* streams, const uint32_t* d_wave_job, const uint32_t* d_job_wave0,
                       const uint16_t* tables, const SyncArrays& A, uint32_t nw, uint32_t n_def, uint32_t* status,
                       uint32_t out_stage) {
  hipLaunchKernelGGL(sync_scan_kernel, dim3(4 * n_def), dim3(256), 0, s, streams, d_job_wave0, A, status);
  PTWM_HIP_TRY_ERR(hipGetLastError());
  if (out_stage <= 8192)
    hipLaunchKernelGGL(sync_write_kernel<8192>, dim3(nw), dim3(kLanes), 0, s, streams, d_wave_job, d_job_wave0, tables,
                       A, status);
  else if (out_stage <= 12288)
    hipLaunchKernelGGL(sync_write_kernel<12288>, dim3(nw), dim3(kLanes), 0, s, streams, d_wave_job, d_job_wave0,
                       tables, A, status);
  else
    hipLaunchKernelGGL(sync_write_kernel<kOutStageMax>, dim3(nw), dim3(kLanes), 0, s, streams, d_wave_job,
                       d_job_wave0, tables, A, status);
  return hipGetLastError();
}

// Fix-pass grid: a lane per wavefront to check, a workgroup per 64.
uint32_t fix_grid(uint32_t nw) { return std::min<uint32_t>((nw + kLanes - 1) / kLanes, 2048u); }

size_t up16(size_t x) { return (x + 15) & ~size_t(15); }

}  // namespace

int64_t decode_jobs_launch(DevCtx& ctx, DecodeJob* hj, size_t n_jobs, ExactRun& run) {
  hipStream_t s = ctx.stream;
  // the kernels write the statuses to host-coherent memory (no copy back);
  // the second half takes the exact path's second run
  PTWM_HIP_TRY(ctx.h_job_status.ensure(2 * n_jobs * sizeof(uint32_t) + 64));
  PTWM_HIP_TRY(ctx.h_status.ensure(n_jobs * sizeof(uint32_t) + 64));
  if (n_jobs == 0) return kOk;
  // Payloads for the parallel path and their slots; output pieces for
  // deferred stored-bytes copies (any job may turn out to be stored).
  std::vector<uint32_t> wave_job, job_wave0, chunk_job, job_chunk0(n_jobs, 0);
  uint64_t subs = 0;
  uint32_t n_def = 0;
  double out_per_wave = 0;  // expected symbols per wavefront, largest over the parallel-path payloads
  // Subsequence size: kSyncSubBitsMax, or, when the launch's wavefronts at
  // that size would not fill the device, smaller in proportion (towards
  // kFillWaves wavefronts), but long enough for about kMinLaneSymbols
  // symbols per lane at the payload's mean code length (a lane that starts
  // off a codeword boundary needs a few codewords to resynchronise).
  constexpr double kFillWaves = 2048, kMinLaneSymbols = 24, kWaveSymbols = 6400;
  double bits_all = 0;
  for (size_t j = 0; j < n_jobs; ++j)
    if (hj[j].codec == kCodecHuffman && hj[j].src_len >= kSyncMinBytes) bits_all += 8.0 * (double)hj[j].src_len;
  const double scale = std::min(1.0, bits_all / (kLanes * (double)kSyncSubBitsMax) / kFillWaves);
  for (size_t j = 0; j < n_jobs; ++j) {
    hj[j].sync_id = 0;
    hj[j].sync_sub0 = 0;
    job_chunk0[j] = (uint32_t)chunk_job.size();
    if (hj[j].dst_len >= kCopyDeferMin) {
      const uint64_t cs = copy_chunk(hj[j].dst_len);
      const uint64_t nc = (hj[j].dst_len + cs - 1) / cs;
      if (chunk_job.size() + nc > 0x7FFFFFFFull) return kInvalidInput;
      chunk_job.insert(chunk_job.end(), nc, (uint32_t)j);
    }
    if (hj[j].codec != kCodecHuffman || hj[j].src_len < kSyncMinBytes) continue;
    const double mean_bits = hj[j].dst_len ? 8.0 * (double)hj[j].src_len / (double)hj[j].dst_len : 8.0;
    const double want = std::max(scale * kSyncSubBitsMax, kMinLaneSymbols * mean_bits);
    uint32_t sb = kSyncSubBitsMin;
    while (sb < kSyncSubBitsMax && sb < want) sb += 64;
    // at most about kWaveSymbols symbols per wavefront, so that the write
    // pass's LDS output staging stays small
    while (sb > kSyncSubBitsMin && kLanes * (double)sb > kWaveSymbols * mean_bits) sb -= 64;
    const uint64_t u = (hj[j].src_len * 8 + sb - 1) / sb + 4;
    const uint64_t waves = (u + kLanes - 1) / kLanes + 4;
    if (subs + u > 0xFFFFFFFFull || wave_job.size() + waves > 0x7FFFFFFFull) continue;
    hj[j].sync_id = ++n_def;
    hj[j].sync_sub0 = (uint32_t)subs;
    hj[j].pad[3] = sb;
    out_per_wave = std::max(out_per_wave, (double)kLanes * sb * (double)hj[j].dst_len / (8.0 * (double)hj[j].src_len));
    job_wave0.push_back((uint32_t)wave_job.size());
    wave_job.insert(wave_job.end(), waves, n_def - 1);
    subs += u;
  }
  const size_t nck = chunk_job.size();
  const uint32_t nw = (uint32_t)wave_job.size();
  // Every argument array in one upload from pinned memory:
  //   jobs | copy sources (zero) | piece -> job | job -> first piece |
  //   [stream records (zero but their job) | wavefront -> payload |
  //    payload -> first wavefront | payload verdicts (zero) | fix-pass
  //    flags (zero)]
  const size_t o_jobs = 0, o_src = up16(n_jobs * sizeof(DecodeJob)), o_cj = o_src + up16(n_jobs * 8),
               o_jc = o_cj + up16(nck * 4), o_str = o_jc + up16(n_jobs * 4),
               o_wj = o_str + up16(4ull * n_def * sizeof(SyncStream)), o_jw = o_wj + up16((size_t)nw * 4),
               o_vd = o_jw + up16((size_t)n_def * 4), o_fl = o_vd + up16((size_t)n_def * 4),
               total = o_fl + up16(4 * kFixQueued);
  PTWM_HIP_TRY(ctx.exact_args.ensure(total));
  PTWM_HIP_TRY(ctx.h_exact_args.ensure(total));
  uint8_t* hb = static_cast<uint8_t*>(ctx.h_exact_args.ptr);
  uint8_t* db = static_cast<uint8_t*>(ctx.exact_args.ptr);
  std::memcpy(hb + o_jobs, hj, n_jobs * sizeof(DecodeJob));
  std::memset(hb + o_src, 0, o_cj - o_src);
  if (nck) std::memcpy(hb + o_cj, chunk_job.data(), nck * 4);
  std::memcpy(hb + o_jc, job_chunk0.data(), n_jobs * 4);
  std::memset(hb + o_str, 0, o_wj - o_str);
  // a payload whose header the exact kernel rejects keeps these records:
  // its verdict then leaves the status the exact kernel set
  SyncStream* hrec = reinterpret_cast<SyncStream*>(hb + o_str);
  for (size_t j = 0; j < n_jobs; ++j)
    if (hj[j].sync_id)
      for (int q = 0; q < 4; ++q) hrec[4ull * (hj[j].sync_id - 1) + q].job = (uint32_t)j;
  if (nw) std::memcpy(hb + o_wj, wave_job.data(), (size_t)nw * 4);
  if (n_def) std::memcpy(hb + o_jw, job_wave0.data(), (size_t)n_def * 4);
  std::memset(hb + o_vd, 0, total - o_vd);
  PTWM_HIP_TRY(hipMemcpyAsync(db, hb, total, hipMemcpyHostToDevice, s));
  const DecodeJob* d_jobs = reinterpret_cast<const DecodeJob*>(db + o_jobs);
  uint64_t* d_copy_src = reinterpret_cast<uint64_t*>(db + o_src);
  const uint32_t* d_chunk_job = reinterpret_cast<const uint32_t*>(db + o_cj);
  const uint32_t* d_job_chunk0 = reinterpret_cast<const uint32_t*>(db + o_jc);
  SyncStream* streams = n_def ? reinterpret_cast<SyncStream*>(db + o_str) : nullptr;
  const uint32_t* d_wave_job = reinterpret_cast<const uint32_t*>(db + o_wj);
  const uint32_t* d_job_wave0 = reinterpret_cast<const uint32_t*>(db + o_jw);
  uint32_t* d_flag = reinterpret_cast<uint32_t*>(db + o_fl);
  uint16_t* tables = nullptr;
  SyncArrays A{};
  // test mode: no look-back, and the queued fix pass marks every stream it
  // touches unsettled, so that the host's extra passes run
  const bool force_unsettled = std::getenv("PTWM_SYNC_FORCE_UNSETTLED") != nullptr;
  if (n_def) {
    PTWM_HIP_TRY(ctx.sync_tables.ensure(2ull * kSyncTableEntries * n_def));
    PTWM_HIP_TRY(ctx.sync_sub.ensure(subs * (8 + 8 + 4) + (uint64_t)nw * (8 + 4) + 64));
    tables = static_cast<uint16_t*>(ctx.sync_tables.ptr);
    uint8_t* sb = static_cast<uint8_t*>(ctx.sync_sub.ptr);
    A.start = reinterpret_cast<uint64_t*>(sb);
    A.exit = A.start + subs;
    A.wave_prefix = A.exit + subs;
    A.count = reinterpret_cast<uint32_t*>(A.wave_prefix + nw);
    A.wave_sum = A.count + subs;
    A.verdict = reinterpret_cast<uint32_t*>(db + o_vd);
    // look-back slots: stale values carry an older epoch; fresh memory is
    // cleared once
    const void* old_pub = ctx.sync_pub.ptr;
    PTWM_HIP_TRY(ctx.sync_pub.ensure((size_t)nw * 8));
    if (ctx.sync_pub.ptr != old_pub) PTWM_HIP_TRY(hipMemsetAsync(ctx.sync_pub.ptr, 0, ctx.sync_pub.cap, s));
    A.pub = static_cast<uint64_t*>(ctx.sync_pub.ptr);
    A.epoch = ++ctx.sync_epoch;
    A.look_back = force_unsettled ? 0u : 1u;
  }
  uint32_t* status = static_cast<uint32_t*>(ctx.h_job_status.ptr);
  run.out_stage = (uint32_t)std::min<double>(kOutStageMax, 1.25 * out_per_wave + 64);
  PTWM_HIP_TRY(launch_decode_exact(d_jobs, status, (uint32_t)n_jobs, streams, tables, d_copy_src, s));
  bool any_zstd = false, any_tans = false;
  for (size_t j = 0; j < n_jobs; ++j) {
    any_zstd |= hj[j].codec == kCodecZstd;
    any_tans |= hj[j].codec == kCodecTans;
  }
  if (any_zstd) PTWM_HIP_TRY(launch_zstd_decode(d_jobs, status, (uint32_t)n_jobs, s));
  if (any_tans) PTWM_HIP_TRY(launch_tans_decode(d_jobs, status, (uint32_t)n_jobs, s));
  // reference rANS payloads are a few long serial chains: they run on the
  // side stream while this stream decodes everything else
  bool any_rans = false;
  for (size_t j = 0; j < n_jobs; ++j) any_rans |= hj[j].codec == kCodecRans;
  if (any_rans) {
    PTWM_HIP_TRY(ctx.ensure_side());
    PTWM_HIP_TRY(hipEventRecord(ctx.side_fork, s));
    PTWM_HIP_TRY(hipStreamWaitEvent(ctx.side_stream, ctx.side_fork, 0));
    // (stored-bytes payloads of rANS jobs are copied by that kernel itself:
    // raw_copy_kernel on this stream does not wait for the side stream)
    PTWM_HIP_TRY(launch_rans_exact(d_jobs, status, (uint32_t)n_jobs, nullptr, ctx.side_stream));
    PTWM_HIP_TRY(hipEventRecord(ctx.side_join, ctx.side_stream));
  }
  bool any_o1sac = false;
  for (size_t j = 0; j < n_jobs; ++j) any_o1sac |= hj[j].codec == kCodecO1sac;
  if (any_o1sac) PTWM_HIP_TRY(launch_o1sac_decode(d_jobs, status, (uint32_t)n_jobs, s));
  const CopyArgs C{d_jobs, d_copy_src, d_chunk_job, d_job_chunk0};
  const uint32_t queued = kFixQueued;
  if (nck && !n_def) {
    hipLaunchKernelGGL(raw_copy_kernel, dim3((uint32_t)nck), dim3(256), 0, s, C);
    PTWM_HIP_TRY(hipGetLastError());
  }
  if (n_def) {
    // the deferred copies ride along as the first pass's last workgroups
    if ((uint64_t)nw + 4ull * nck > 0xFFFFFFFFull) return kInvalidInput;
    hipLaunchKernelGGL(sync_pass_kernel, dim3(nw + 4 * (uint32_t)nck), dim3(kLanes), 0, s, streams, d_wave_job,
                       d_job_wave0, tables, A, nw, C);
    PTWM_HIP_TRY(hipGetLastError());
    for (uint32_t k = 0; k < queued; ++k) {
      hipLaunchKernelGGL(sync_fix_kernel, dim3(fix_grid(nw)), dim3(kLanes), 0, s, streams, d_wave_job, d_job_wave0,
                         tables, A, nw, k ? d_flag + k - 1 : nullptr, d_flag + k,
                         k + 1 < queued ? 0u : force_unsettled ? 2u : 1u);
      PTWM_HIP_TRY(hipGetLastError());
    }
    PTWM_HIP_TRY(sync_finish(s, streams, d_wave_job, d_job_wave0, tables, A, nw, n_def, status, run.out_stage));
  }
  if (any_rans) PTWM_HIP_TRY(hipStreamWaitEvent(s, ctx.side_join, 0));
  run.jobs = d_jobs;
  run.status = status;
  run.streams = streams;
  run.tables = tables;
  run.A = A;
  run.wave_job = d_wave_job;
  run.job_wave0 = d_job_wave0;
  run.nw = nw;
  run.n_def = n_def;
  return kOk;
}

int64_t decode_jobs_complete(DevCtx& ctx, DecodeJob* hj, size_t n_jobs, ExactRun& run, bool& rewritten) {
  hipStream_t s = ctx.stream;
  rewritten = false;
  uint32_t* const status = run.status;
  volatile uint32_t* const hs = status;  // host-coherent: read after the stream is synchronised
  SyncStream* streams = run.streams;
  const uint16_t* tables = run.tables;
  const SyncArrays& A = run.A;
  const uint32_t* d_wave_job = run.wave_job;
  const uint32_t* d_job_wave0 = run.job_wave0;
  const uint32_t nw = run.nw, n_def = run.n_def;
  // payloads whose wavefront boundaries the queued passes did not settle:
  // more fix passes until none changes (host-checked batches), then the
  // offsets, the write and the check again
  bool unsettled = false;
  for (size_t j = 0; j < n_jobs; ++j) unsettled |= hs[j] == kStUnsettled;
  if (unsettled) {
    ++ctx.sync_extra_rounds;
    rewritten = true;
    constexpr uint32_t kBatch = 4;
    PTWM_HIP_TRY(ctx.sync_waves.ensure(4 * kBatch + 64));
    uint32_t* fl = static_cast<uint32_t*>(ctx.sync_waves.ptr);
    PTWM_HIP_TRY(ctx.h_small.ensure(64));
    volatile uint32_t* h_flag = static_cast<uint32_t*>(ctx.h_small.ptr);
    bool settled = false;
    for (uint32_t pass = 0; pass < kMaxFixPasses && !settled; pass += kBatch) {
      PTWM_HIP_TRY(hipMemsetAsync(fl, 0, 4 * kBatch, s));
      for (uint32_t k = 0; k < kBatch; ++k) {
        hipLaunchKernelGGL(sync_fix_kernel, dim3(fix_grid(nw)), dim3(kLanes), 0, s, streams, d_wave_job, d_job_wave0,
                           tables, A, nw, k ? fl + k - 1 : nullptr, fl + k, 0u);
        PTWM_HIP_TRY(hipGetLastError());
      }
      PTWM_HIP_TRY(hipMemcpyAsync(const_cast<uint32_t*>(h_flag), fl, 4 * kBatch, hipMemcpyDeviceToHost, s));
      PTWM_HIP_TRY(hipStreamSynchronize(s));
      for (uint32_t k = 0; k < kBatch; ++k) settled |= h_flag[k] == 0;
    }
    if (!settled) {
      // still moving after kMaxFixPasses: the exact path decodes them
      for (size_t j = 0; j < n_jobs; ++j)
        if (hs[j] == kStUnsettled) hs[j] = kStFallback;
    } else {
      // the streams' unsettled marks and the verdicts are cleared; jobs
      // already final keep their status (the write of a settled payload
      // writes the same bytes)
      std::vector<uint32_t> keep(n_jobs);
      for (size_t j = 0; j < n_jobs; ++j) keep[j] = hs[j];
      hipLaunchKernelGGL(clear_unsettled_kernel, dim3((4 * n_def + 255) / 256), dim3(256), 0, s, streams, A.verdict,
                         n_def);
      PTWM_HIP_TRY(hipGetLastError());
      for (size_t j = 0; j < n_jobs; ++j)
        if (keep[j] == kStUnsettled) keep[j] = kStDeferred;
      for (size_t j = 0; j < n_jobs; ++j) hs[j] = keep[j];
      PTWM_HIP_TRY(sync_finish(s, streams, d_wave_job, d_job_wave0, tables, A, nw, n_def, status, run.out_stage));
      PTWM_HIP_TRY(hipStreamSynchronize(s));
      for (size_t j = 0; j < n_jobs; ++j)
        if (keep[j] != kStDeferred) hs[j] = keep[j];
    }
  }
  // payloads the parallel path declined (or did not settle) go to the exact path
  std::vector<DecodeJob> again;
  std::vector<size_t> again_idx;
  for (size_t j = 0; j < n_jobs; ++j) {
    if (hj[j].sync_id && hs[j] == kStOk) ++ctx.sync_accepted;
    if (hs[j] == kStFallback || hs[j] == kStDeferred || hs[j] == kStUnsettled) {
      if (hj[j].sync_id) ++ctx.sync_fallbacks;
      DecodeJob J = hj[j];
      J.sync_id = 0;
      J.sync_sub0 = 0;
      again.push_back(J);
      again_idx.push_back(j);
    }
  }
  if (!again.empty()) {
    rewritten = true;
    const size_t na = again.size();
    PTWM_HIP_TRY(ctx.jobs.ensure(na * sizeof(DecodeJob) + 64));
    PTWM_HIP_TRY(hipMemcpyAsync(ctx.jobs.ptr, again.data(), na * sizeof(DecodeJob), hipMemcpyHostToDevice, s));
    PTWM_HIP_TRY(launch_decode_exact(static_cast<const DecodeJob*>(ctx.jobs.ptr), status + n_jobs, (uint32_t)na,
                                     nullptr, nullptr, nullptr, s));
    PTWM_HIP_TRY(hipStreamSynchronize(s));
    for (size_t i = 0; i < na; ++i) hs[again_idx[i]] = hs[n_jobs + i];
  }
  uint32_t* const out = static_cast<uint32_t*>(ctx.h_status.ptr);
  for (size_t j = 0; j < n_jobs; ++j) out[j] = hs[j];
  return kOk;
}

int64_t decode_jobs(DevCtx& ctx, DecodeJob* hj, size_t n_jobs) {
  ExactRun run;
  int64_t rc = decode_jobs_launch(ctx, hj, n_jobs, run);
  if (rc != kOk || n_jobs == 0) return rc;
  PTWM_HIP_TRY(hipStreamSynchronize(ctx.stream));
  bool rewritten = false;
  return decode_jobs_complete(ctx, hj, n_jobs, run, rewritten);
}

}  // namespace ptwm
