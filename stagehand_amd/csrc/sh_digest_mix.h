// Chunk-digest arithmetic shared by the digest kernels (sh_digest.hip, built into the
// library's embedded code object) and the host digest (sh_digest.cpp): the position key, the two
// bijective 32-bit mixers and the per-word update. The definition of a digest is in sh_digest.cpp.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr uint32_t kKey = 0x9E3779B9u;  // word j's key is j * kKey mod 2^32
constexpr uint32_t kDigestThreads = 256;

// MurmurHash3's 32-bit finalizer (Austin Appleby, public domain).
__host__ __device__ inline uint32_t mix_f(uint32_t x) {
  x ^= x >> 16;
  x *= 0x85EBCA6Bu;
  x ^= x >> 13;
  x *= 0xC2B2AE35u;
  return x ^ (x >> 16);
}

// "lowbias32" (Chris Wellons, hash-prospector, public domain): the same xorshift-multiply form
// with other shifts and multipliers.
__host__ __device__ inline uint32_t mix_g(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7FEB352Du;
  x ^= x >> 15;
  x *= 0x846CA68Bu;
  return x ^ (x >> 16);
}

// Word w at position j (its byte offset / 8) with key k = j * kKey: its halves l, h keyed, then
// sa += f(l ^ k) + f(h ^ k) * 2^32 and sb += g(l ^ k) + g(h ^ k) * 2^32 (mod 2^64).
__host__ __device__ inline void add_keyed(uint64_t w, uint32_t k, uint64_t& sa, uint64_t& sb) {
  const uint32_t l = (uint32_t)w ^ k, h = (uint32_t)(w >> 32) ^ k;
  sa += (uint64_t)mix_f(l) | ((uint64_t)mix_f(h) << 32);
  sb += (uint64_t)mix_g(l) | ((uint64_t)mix_g(h) << 32);
}

__host__ __device__ inline void add_word(uint64_t w, uint64_t j, uint64_t& sa, uint64_t& sb) {
  add_keyed(w, (uint32_t)j * kKey, sa, sb);
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
