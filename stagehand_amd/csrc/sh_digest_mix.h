// Chunk-digest arithmetic shared by the digest kernels (sh_digest.hip, built into the
// library's embedded code object) and the host digest (sh_digest.cpp): the keys, the two
// bijective mixers and the per-word update. The definition of a digest is in sh_digest.cpp.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr uint64_t kKeyA = 0x9E3779B97F4A7C15ull;
constexpr uint64_t kKeyB = 0xC2B2AE3D27D4EB4Full;
constexpr uint64_t kKeyC = 0x165667B19E3779F9ull;
constexpr uint32_t kDigestThreads = 256;

__host__ __device__ inline uint64_t mix_a(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__host__ __device__ inline uint64_t mix_b(uint64_t z) {
  z = (z ^ (z >> 33)) * 0xFF51AFD7ED558CCDull;
  z = (z ^ (z >> 29)) * 0xC4CEB9FE1A85EC53ull;
  return z ^ (z >> 32);
}

__host__ __device__ inline void add_word(uint64_t w, uint64_t j, uint64_t& sa, uint64_t& sb) {
  sa += mix_a(w ^ (j * kKeyA));
  sb += mix_b(w ^ (j * kKeyB) ^ kKeyC);
}

// The partial words after the last whole 16 bytes of [off, e): at most 15 bytes.
__host__ __device__ inline void add_tail(const uint8_t* buf, uint64_t off, uint64_t e, uint64_t& sa, uint64_t& sb) {
  while (off < e) {
    uint64_t w = 0;
    const uint64_t n = (e - off) < 8 ? (e - off) : 8;
    for (uint64_t k = 0; k < n; ++k) w |= (uint64_t)buf[off + k] << (8 * k);
    add_word(w, off >> 3, sa, sb);
    off += 8;
  }
}

}  // namespace
