// blake3_host.h -- BLAKE3 hash (32 bytes) on the host.
#pragma once

#include <array>
#include <cstddef>
#include <cstdint>

namespace ptwm {

void blake3_hash(const uint8_t* data, size_t len, uint8_t out[32]);

}  // namespace ptwm
