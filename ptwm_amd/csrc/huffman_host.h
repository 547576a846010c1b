// huffman_host.h -- host-side canonical Huffman table construction.
#pragma once

#include <cstdint>

namespace ptwm {

constexpr int kHufMaxBits = 11;  // MAX_TABLE_LOG (entropy/huffman/tree.rs:5)

// Code lengths from a histogram (tree.rs:19-85 + enforce_max_code_length
// :212-242 at max_len, the reference encoder's 11 by default).  Returns false
// when every count is zero.
bool huf_lengths_from_freqs(const uint32_t freqs[256], uint8_t lengths[256], int max_len = kHufMaxBits);

// huff_ilv's code lengths: the limit is 6 when every symbol is < 16 (nibble
// planes, so that every pair of codes fits one 12-bit decode lookup), else 11.
constexpr int kIlvNibbleMaxLen = 6;
bool ilv_lengths_from_freqs(const uint32_t freqs[256], uint8_t lengths[256]);

// Canonical codes (tree.rs:102-177): fills bit-reversed codes, returns
// max_bits or 0 if the lengths do not form a valid prefix code.
int huf_canonical(const uint8_t lengths[256], uint16_t rev_codes[256]);

// Weights header (weights.rs:8-32) into out (<= 130 bytes); returns its length.
int huf_encode_weights(const uint8_t lengths[256], uint8_t* out);

// rANS frequency normalisation of the reference (rans/compress.rs:72-122):
// 11-bit frequencies summing to 2048, at least 1 for every present symbol,
// the excess or deficit absorbed by the first most frequent symbol.
// Returns false when that fails (the reference then stores the plane).
bool rans_normalize_freqs(const uint32_t raw[256], uint16_t f[256], uint16_t cum[256], int* max_sym_out);

}  // namespace ptwm
