// xxh64_host.cpp -- XXH64 (seed 0), streaming, on one host core.
// XXH64 itself follows the published specification (Collet, xxHash
// "XXH64 algorithm description"): primes P1..P5, round(acc, x) =
// rotl(acc + x P2, 31) P1, four lanes seeded P1 + P2, P2, 0, -P1, then the
// merge, length, tail (8-, 4- and 1-byte steps) and avalanche.
#include "xxh64_host.h"

#include <algorithm>
#include <cstring>

namespace ptwm {

namespace {

constexpr uint64_t kP1 = 0x9E3779B185EBCA87ull, kP2 = 0xC2B2AE3D27D4EB4Full, kP3 = 0x165667B19E3779F9ull,
                   kP4 = 0x85EBCA77C2B2AE63ull, kP5 = 0x27D4EB2F165667C5ull;

inline uint64_t rotl(uint64_t x, int r) { return (x << r) | (x >> (64 - r)); }
inline uint64_t rd64(const uint8_t* p) {
  uint64_t v;
  std::memcpy(&v, p, 8);
  return v;
}
inline uint32_t rd32(const uint8_t* p) {
  uint32_t v;
  std::memcpy(&v, p, 4);
  return v;
}
inline uint64_t round1(uint64_t acc, uint64_t x) { return rotl(acc + x * kP2, 31) * kP1; }
inline uint64_t merge1(uint64_t h, uint64_t v) { return (h ^ round1(0, v)) * kP1 + kP4; }

}  // namespace

void Xxh64::update(const uint8_t* p, size_t n) {
  total += n;
  if (buf_len) {  // complete a stripe held back by the previous update
    const size_t k = std::min<size_t>(32 - buf_len, n);
    std::memcpy(buf + buf_len, p, k);
    buf_len += (uint32_t)k;
    p += k;
    n -= k;
    if (buf_len < 32) return;
    for (int i = 0; i < 4; ++i) v[i] = round1(v[i], rd64(buf + 8 * i));
    buf_len = 0;
  }
  uint64_t a = v[0], b = v[1], c = v[2], d = v[3];
  for (; n >= 32; n -= 32, p += 32) {
    a = round1(a, rd64(p));
    b = round1(b, rd64(p + 8));
    c = round1(c, rd64(p + 16));
    d = round1(d, rd64(p + 24));
  }
  v[0] = a;
  v[1] = b;
  v[2] = c;
  v[3] = d;
  if (n) {
    std::memcpy(buf, p, n);
    buf_len = (uint32_t)n;
  }
}

uint64_t Xxh64::digest() const {
  uint64_t h;
  if (total >= 32) {
    h = rotl(v[0], 1) + rotl(v[1], 7) + rotl(v[2], 12) + rotl(v[3], 18);
    for (int i = 0; i < 4; ++i) h = merge1(h, v[i]);
  } else {
    h = kP5;  // seed 0
  }
  h += total;
  const uint8_t* p = buf;
  uint32_t rest = buf_len;
  for (; rest >= 8; rest -= 8, p += 8) h = rotl(h ^ round1(0, rd64(p)), 27) * kP1 + kP4;
  if (rest >= 4) {
    h = rotl(h ^ ((uint64_t)rd32(p) * kP1), 23) * kP2 + kP3;
    rest -= 4;
    p += 4;
  }
  for (; rest; --rest, ++p) h = rotl(h ^ ((uint64_t)*p * kP5), 11) * kP1;
  h ^= h >> 33;
  h *= kP2;
  h ^= h >> 29;
  h *= kP3;
  h ^= h >> 32;
  return h;
}

void Xxh64::reset() {
  v[0] = kP1 + kP2;
  v[1] = kP2;
  v[2] = 0;
  v[3] = 0 - kP1;
  total = 0;
  buf_len = 0;
}

}  // namespace ptwm
