// xxh64_host.h -- streaming XXH64 (seed 0) on the host: the tensor payload
// hash of container.rs:2185-2194 and compact.rs:441-445 and the PTWC
// meta_xxh64 of ptwc.rs:75-95 (xxhash-rust 0.8.18 xxh64).  Plain C++, no
// HIP dependency, so the container parser builds on its own.
#pragma once

#include <cstddef>
#include <cstdint>

namespace ptwm {

struct Xxh64 {
  uint64_t v[4];
  uint64_t total;
  uint8_t buf[32];
  uint32_t buf_len;
  void reset();
  void update(const uint8_t* p, size_t n);
  uint64_t digest() const;
};

inline uint64_t xxh64_once(const uint8_t* p, size_t n) {
  Xxh64 h;
  h.reset();
  h.update(p, n);
  return h.digest();
}

}  // namespace ptwm
