// blake3_host.cpp -- BLAKE3 (32-byte hash mode) on the host, from the
// published specification (O'Connor, Aumasson, Neves, Wilcox-O'Hearn,
// "BLAKE3: one function, fast everywhere", 2020): 1 KiB chunks of 64-byte
// blocks compressed with the 7-round function, chunk chaining values merged
// pairwise into a binary tree whose left subtrees are complete, the root
// compressed with the ROOT flag.  The legacy container header commits to its
// Extension Table with it (header.rs extension_table_hash).
#include "blake3_host.h"

#include <cstring>
#include <vector>

namespace ptwm {

namespace {

constexpr uint32_t kIv[8] = {0x6A09E667u, 0xBB67AE85u, 0x3C6EF372u, 0xA54FF53Au,
                             0x510E527Fu, 0x9B05688Cu, 0x1F83D9ABu, 0x5BE0CD19u};
constexpr uint8_t kPerm[16] = {2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8};
constexpr uint32_t kChunkStart = 1, kChunkEnd = 2, kParent = 4, kRoot = 8;
constexpr size_t kBlock = 64, kChunk = 1024;

inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

inline void g(uint32_t* s, int a, int b, int c, int d, uint32_t mx, uint32_t my) {
  s[a] = s[a] + s[b] + mx;
  s[d] = rotr(s[d] ^ s[a], 16);
  s[c] = s[c] + s[d];
  s[b] = rotr(s[b] ^ s[c], 12);
  s[a] = s[a] + s[b] + my;
  s[d] = rotr(s[d] ^ s[a], 8);
  s[c] = s[c] + s[d];
  s[b] = rotr(s[b] ^ s[c], 7);
}

// The compression function: chaining value, 16 message words, block counter,
// block length and flags in; the first eight output words out.
void compress(const uint32_t cv[8], const uint32_t block[16], uint64_t counter, uint32_t len, uint32_t flags,
              uint32_t out[8]) {
  uint32_t s[16] = {cv[0],  cv[1],  cv[2],  cv[3],  cv[4],          cv[5],                    cv[6], cv[7],
                    kIv[0], kIv[1], kIv[2], kIv[3], (uint32_t)counter, (uint32_t)(counter >> 32), len,  flags};
  uint32_t m[16];
  std::memcpy(m, block, sizeof m);
  for (int round = 0; round < 7; ++round) {
    g(s, 0, 4, 8, 12, m[0], m[1]);
    g(s, 1, 5, 9, 13, m[2], m[3]);
    g(s, 2, 6, 10, 14, m[4], m[5]);
    g(s, 3, 7, 11, 15, m[6], m[7]);
    g(s, 0, 5, 10, 15, m[8], m[9]);
    g(s, 1, 6, 11, 12, m[10], m[11]);
    g(s, 2, 7, 8, 13, m[12], m[13]);
    g(s, 3, 4, 9, 14, m[14], m[15]);
    if (round < 6) {
      uint32_t t[16];
      for (int i = 0; i < 16; ++i) t[i] = m[kPerm[i]];
      std::memcpy(m, t, sizeof m);
    }
  }
  for (int i = 0; i < 8; ++i) out[i] = s[i] ^ s[i + 8];
}

void words(const uint8_t* p, size_t n, uint32_t w[16]) {  // a block, zero-padded, little endian
  uint8_t b[kBlock] = {0};
  std::memcpy(b, p, n);
  for (int i = 0; i < 16; ++i)
    w[i] = (uint32_t)b[4 * i] | ((uint32_t)b[4 * i + 1] << 8) | ((uint32_t)b[4 * i + 2] << 16) |
           ((uint32_t)b[4 * i + 3] << 24);
}

// What the last compression of a node takes, so that the root can be
// compressed again with ROOT.
struct Node {
  uint32_t cv[8];
  uint32_t block[16];
  uint64_t counter;
  uint32_t len, flags;
  void chaining_value(uint32_t out[8]) const { compress(cv, block, counter, len, flags, out); }
};

// chunk `index` of n bytes (0 < n <= 1024, or 0 for the empty input)
Node chunk_node(const uint8_t* p, size_t n, uint64_t index) {
  Node nd;
  std::memcpy(nd.cv, kIv, sizeof kIv);
  const size_t blocks = n ? (n + kBlock - 1) / kBlock : 1;
  for (size_t b = 0; b < blocks; ++b) {
    const size_t len = b + 1 < blocks ? kBlock : n - b * kBlock;
    uint32_t w[16];
    words(p + b * kBlock, len, w);
    const uint32_t flags = (b == 0 ? kChunkStart : 0) | (b + 1 == blocks ? kChunkEnd : 0);
    if (b + 1 < blocks) {
      uint32_t next[8];
      compress(nd.cv, w, index, (uint32_t)len, flags, next);
      std::memcpy(nd.cv, next, sizeof next);
    } else {
      std::memcpy(nd.block, w, sizeof w);
      nd.counter = index;
      nd.len = (uint32_t)len;
      nd.flags = flags;
    }
  }
  return nd;
}

Node parent_node(const uint32_t left[8], const uint32_t right[8]) {
  Node nd;
  std::memcpy(nd.cv, kIv, sizeof kIv);
  std::memcpy(nd.block, left, 32);
  std::memcpy(nd.block + 8, right, 32);
  nd.counter = 0;
  nd.len = kBlock;
  nd.flags = kParent;
  return nd;
}

}  // namespace

void blake3_hash(const uint8_t* data, size_t len, uint8_t out[32]) {
  const size_t chunks = len ? (len + kChunk - 1) / kChunk : 1;
  std::vector<std::array<uint32_t, 8>> stack;
  Node last{};
  for (size_t c = 0; c < chunks; ++c) {
    const size_t n = c + 1 < chunks ? kChunk : len - c * kChunk;
    const Node nd = chunk_node(data + c * kChunk, n, c);
    if (c + 1 == chunks) {
      last = nd;
      break;
    }
    // push the chunk's chaining value, merging complete subtrees: after
    // chunk c the stack holds one value per set bit of c + 1
    std::array<uint32_t, 8> cv;
    nd.chaining_value(cv.data());
    uint64_t total = c + 1;
    while ((total & 1) == 0) {
      std::array<uint32_t, 8> merged;
      parent_node(stack.back().data(), cv.data()).chaining_value(merged.data());
      stack.pop_back();
      cv = merged;
      total >>= 1;
    }
    stack.push_back(cv);
  }
  while (!stack.empty()) {
    uint32_t right[8];
    last.chaining_value(right);
    last = parent_node(stack.back().data(), right);
    stack.pop_back();
  }
  uint32_t h[8];
  compress(last.cv, last.block, last.counter, last.len, last.flags | kRoot, h);
  for (int i = 0; i < 8; ++i)
    for (int k = 0; k < 4; ++k) out[4 * i + k] = (uint8_t)(h[i] >> (8 * k));
}

}  // namespace ptwm
