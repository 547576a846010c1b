// huffman_host.cpp -- canonical Huffman code construction on the host.
//
// Builds exactly the code lengths and canonical codes of the reference
// encoder (crates/ptwm-core/src/entropy/huffman/tree.rs:19-177) from a
// 256-bin histogram, plus the weights header (weights.rs:8-32).  Only the
// 256-symbol table is built here; all per-symbol work runs on the GPU.
//
// Tie-breaking follows tree.rs:51-65: nodes are merged in ascending
// (frequency, id) order, leaves take ids 0..n-1 in ascending symbol order and
// internal nodes the following ids in creation order.  Internal frequencies
// never decrease in creation order, so two FIFO queues (sorted leaves,
// internal nodes) pop in exactly the order of the reference's binary heap.
#include "huffman_host.h"

#include <algorithm>
#include <cstring>

namespace ptwm {

bool huf_lengths_from_freqs(const uint32_t freqs[256], uint8_t lengths[256], int max_len) {
  if (max_len < 1 || max_len > kHufMaxBits) return false;
  std::memset(lengths, 0, 256);
  int sym[256];
  int n = 0;
  for (int i = 0; i < 256; ++i)
    if (freqs[i]) sym[n++] = i;
  if (n == 0) return false;
  if (n == 1) {
    lengths[sym[0]] = 1;
    return true;
  }
  // leaves sorted by (freq, id); ids are ascending symbol order already
  int order[256];
  for (int i = 0; i < n; ++i) order[i] = i;
  std::stable_sort(order, order + n, [&](int a, int b) { return freqs[sym[a]] < freqs[sym[b]]; });
  uint64_t f[512];
  int parent[512];
  for (int i = 0; i < n; ++i) f[i] = freqs[sym[i]];
  int li = 0;              // next leaf in `order`
  int qi = n, qe = n;      // internal-node FIFO [qi, qe)
  auto take = [&]() -> int {
    // pop the smaller (freq, id); leaves have smaller ids than internal nodes
    bool leaf_ok = li < n;
    bool int_ok = qi < qe;
    if (leaf_ok && (!int_ok || f[order[li]] <= f[qi])) return order[li++];
    return qi++;
  };
  while ((n - li) + (qe - qi) > 1) {
    int a = take();
    int b = take();
    f[qe] = f[a] + f[b];
    parent[a] = qe;
    parent[b] = qe;
    ++qe;
  }
  const int root = qe - 1;
  // depth = number of edges to the root (DFS in tree.rs:66-81 gives the same)
  int depth[512];
  depth[root] = 0;
  for (int id = root - 1; id >= 0; --id) {
    int d = depth[parent[id]] + 1;
    depth[id] = d > 255 ? 255 : d;
  }
  for (int i = 0; i < n; ++i) lengths[sym[i]] = (uint8_t)depth[i];
  // enforce_max_code_length (tree.rs:212-242)
  bool clamped = false;
  for (int s = 0; s < 256; ++s)
    if (lengths[s] > max_len) {
      lengths[s] = (uint8_t)max_len;
      clamped = true;
    }
  if (clamped) {
    const uint32_t cap = 1u << max_len;
    for (;;) {
      uint32_t kraft = 0;
      for (int s = 0; s < 256; ++s)
        if (lengths[s]) kraft += 1u << (max_len - lengths[s]);
      if (kraft <= cap) break;
      int victim = -1;
      for (int s = 0; s < 256; ++s)
        if (lengths[s] > 0 && lengths[s] < max_len && (victim < 0 || lengths[s] < lengths[victim])) victim = s;
      if (victim < 0) break;
      lengths[victim]++;
    }
  }
  return true;
}

bool ilv_lengths_from_freqs(const uint32_t freqs[256], uint8_t lengths[256]) {
  bool nibble = true;
  for (int s = 16; s < 256; ++s)
    if (freqs[s]) nibble = false;
  return huf_lengths_from_freqs(freqs, lengths, nibble ? kIlvNibbleMaxLen : kHufMaxBits);
}

int huf_canonical(const uint8_t lengths[256], uint16_t rev_codes[256]) {
  int max_bits = 0;
  for (int s = 0; s < 256; ++s) max_bits = std::max(max_bits, (int)lengths[s]);
  if (max_bits < 1) max_bits = 1;
  if (max_bits > kHufMaxBits) return 0;
  uint32_t counts[kHufMaxBits + 1] = {0};
  uint32_t total = 0;
  for (int s = 0; s < 256; ++s)
    if (lengths[s]) {
      counts[lengths[s]]++;
      total++;
    }
  if (!total) return 0;
  uint32_t next[kHufMaxBits + 1] = {0};
  uint32_t code = 0;
  for (int b = 1; b <= max_bits; ++b) {
    code = (code + counts[b - 1]) << 1;
    if (code > (1u << b)) return 0;
    next[b] = code;
  }
  for (int s = 0; s < 256; ++s) {
    int l = lengths[s];
    if (!l) {
      rev_codes[s] = 0;
      continue;
    }
    uint32_t c = next[l]++;
    if (c >= (1u << l)) return 0;
    uint32_t r = 0;
    for (int k = 0; k < l; ++k) r |= ((c >> k) & 1u) << (l - 1 - k);
    rev_codes[s] = (uint16_t)r;
  }
  return max_bits;
}

int huf_encode_weights(const uint8_t lengths[256], uint8_t* out) {
  int n = 0;
  for (int s = 0; s < 256; ++s)
    if (lengths[s]) n = s + 1;
  if (n == 0) return -1;
  int o = 0;
  if (n <= 127) {
    out[o++] = (uint8_t)(0x80 | n);
  } else {
    out[o++] = 0x80;
    out[o++] = (uint8_t)n;  // 256 wraps to 0
  }
  for (int i = 0; i < n; i += 2) {
    uint8_t lo = lengths[i] & 0x0F;
    uint8_t hi = (i + 1 < n) ? (lengths[i + 1] & 0x0F) : 0;
    out[o++] = (uint8_t)(lo | (hi << 4));
  }
  return o;
}

constexpr uint32_t kRansNormScale = 2048;  // 1 << PROB_BITS (rans/compress.rs)

// normalize_freqs (rans/compress.rs:72-122): returns false when it fails.
bool rans_normalize_freqs(const uint32_t raw[256], uint16_t f[256], uint16_t cum[256], int* max_sym_out) {
  uint64_t total = 0;
  for (int i = 0; i < 256; ++i) total += raw[i];
  std::memset(f, 0, 512);
  std::memset(cum, 0, 512);
  if (total == 0) return false;
  uint32_t assigned = 0;
  int max_sym = 0, max_freq_sym = 0;
  for (int i = 0; i < 256; ++i) {
    if (raw[i] > 0) {
      uint64_t v = ((uint64_t)raw[i] * kRansNormScale) / total;
      if (v < 1) v = 1;
      f[i] = (uint16_t)v;
      assigned += f[i];
      max_sym = i;
      if (raw[i] > raw[max_freq_sym]) max_freq_sym = i;
    }
  }
  if (assigned > kRansNormScale) {
    const uint32_t excess = assigned - kRansNormScale;
    if ((uint32_t)f[max_freq_sym] > excess) f[max_freq_sym] = (uint16_t)(f[max_freq_sym] - excess);
    else return false;
  } else if (assigned < kRansNormScale) {
    f[max_freq_sym] = (uint16_t)(f[max_freq_sym] + (kRansNormScale - assigned));
  }
  uint16_t run = 0;
  for (int i = 0; i <= max_sym; ++i) {
    cum[i] = run;
    run = (uint16_t)(run + f[i]);
  }
  *max_sym_out = max_sym;
  return true;
}

}  // namespace ptwm

extern "C" int64_t ptwm_mi355x_huffman_code_lengths(const uint32_t* freqs, uint8_t* lengths_out) {
  if (!freqs || !lengths_out) return -1;
  return ptwm::huf_lengths_from_freqs(freqs, lengths_out) ? 0 : -1;
}
