// Chunk digests of device buffers: which chunks of a block changed on the device.
//
// The reference's training eviction copies a module-backed block's parameters back to host
// memory whole (`param.data.to("cpu")`, src/stagehand/scheduler.py:1216-1226, 1348-1366),
// though most of those bytes are frozen weights that its last load brought from the same
// host memory and nothing has written since. Here a block loaded from its pinned home buffer
// gets a digest per chunk on the device right after the load (sh_loader, the load request's
// `digest`); at its eviction the save-back engine's worker takes the digests again
// (sh_block_changed) and copies back only the chunks whose digests differ. The home buffer
// then holds exactly the device's bytes, as after the full copy; the device pays two reads of
// the block from HBM (about 0.1 ms each for a 740 MB block) to save the PCIe copy.
//
// The digest of chunk [b, e) of a buffer is a pair of 64-bit sums, over every 8-byte word
// w_j of the chunk (j = byte offset in the buffer / 8; the last partial word of the buffer is
// zero-padded), of
//   A: mix_a(w_j ^ (j * kKeyA))    and    B: mix_b(w_j ^ (j * kKeyB) ^ kKeyC),
// modulo 2^64. mix_a is the output function of SplitMix64 (Steele, Lea and Flood, "Fast
// splittable pseudorandom number generators", OOPSLA 2014); mix_b has the same
// xorshift-multiply form with other shifts and the odd multipliers of MurmurHash3's 64-bit
// finalizer. Each step is a bijection of 64-bit words (an xorshift by at least half the width,
// a multiply by an odd constant, an xor with a key fixed by the position), so a change of one
// word changes both sums. Several changed words leave a chunk's digest unchanged only if their
// mixed differences cancel in both sums at once, which for two unrelated mixers is a chance of
// about 2^-128. The sums commute, so the digest does not depend on how the words are spread
// over threads.

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>

#include "sh_internal.h"
#include "stagehand_native.h"

namespace {

constexpr uint64_t kKeyA = 0x9E3779B97F4A7C15ull;
constexpr uint64_t kKeyB = 0xC2B2AE3D27D4EB4Full;
constexpr uint64_t kKeyC = 0x165667B19E3779F9ull;
constexpr uint32_t kDigestThreads = 256;
constexpr uint64_t kMaxChunks = 0x7FFFFFFFull;  // one workgroup per chunk, a 1-D grid

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

// One workgroup per chunk. COMPARE: changed[c] = 1 when the chunk's digest differs from
// digests[2c], digests[2c + 1], else 0; otherwise the digest is written there.
template <bool COMPARE>
__global__ __launch_bounds__(kDigestThreads) void digest_kernel(const uint8_t* __restrict__ buf, uint64_t bytes,
                                                                uint64_t chunk, uint64_t* __restrict__ digests,
                                                                uint8_t* __restrict__ changed) {
  const uint64_t c = blockIdx.x;
  const uint64_t b = c * chunk;
  const uint64_t e = (bytes - b > chunk) ? b + chunk : bytes;
  const uint64_t n16 = (e - b) / 16;
  uint64_t sa = 0, sb = 0;
  // The position keys j*kKeyA and j*kKeyB of the thread's words advance by a constant each
  // iteration (mod 2^64), so they are added rather than multiplied per word: the kernel is bound
  // by its 64-bit multiplies (each a v_mad_u64_u32 and two v_mul_lo_u32), and the keys were 2 of
  // the 6 per word (measured on MI355X: 0.164 -> 0.147 ms over 740 MiB).
  constexpr uint64_t kStep = 2ull * kDigestThreads;  // words between a thread's iterations
  const uint64_t j0 = (b >> 3) + 2ull * threadIdx.x;
  uint64_t ka = j0 * kKeyA, kb = j0 * kKeyB;
#pragma unroll 4
  for (uint64_t i = threadIdx.x; i < n16; i += kDigestThreads) {
    uint64_t w[2];
    __builtin_memcpy(w, buf + b + i * 16, 16);
    sa += mix_a(w[0] ^ ka);
    sb += mix_b(w[0] ^ kb ^ kKeyC);
    sa += mix_a(w[1] ^ (ka + kKeyA));
    sb += mix_b(w[1] ^ (kb + kKeyB) ^ kKeyC);
    ka += kStep * kKeyA;
    kb += kStep * kKeyB;
  }
  if (threadIdx.x == 0) add_tail(buf, b + n16 * 16, e, sa, sb);
  // workgroup sum: within each wavefront, then across the four through LDS
  for (int m = 32; m >= 1; m >>= 1) {
    sa += __shfl_xor(sa, m);
    sb += __shfl_xor(sb, m);
  }
  __shared__ uint64_t part[2][kDigestThreads / 64];
  const uint32_t wave = threadIdx.x / 64;
  if ((threadIdx.x & 63) == 0) {
    part[0][wave] = sa;
    part[1][wave] = sb;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t ta = 0, tb = 0;
    for (uint32_t k = 0; k < kDigestThreads / 64; ++k) {
      ta += part[0][k];
      tb += part[1][k];
    }
    if (COMPARE) {
      changed[c] = (ta != digests[2 * c] || tb != digests[2 * c + 1]) ? 1 : 0;
    } else {
      digests[2 * c] = ta;
      digests[2 * c + 1] = tb;
    }
  }
}

uint64_t chunks_of(uint64_t bytes, uint32_t chunk_bytes) {
  return bytes / chunk_bytes + (bytes % chunk_bytes != 0 ? 1 : 0);
}

int check_args(const void* buf, uint64_t bytes, uint32_t chunk_bytes, const void* digests, const char* who) {
  if (chunk_bytes == 0 || chunk_bytes % 16 != 0)
    return sh::fail(SH_ERR_INVALID, "%s: chunk_bytes %u is not a positive multiple of 16", who, chunk_bytes);
  if (bytes > 0 && (buf == nullptr || digests == nullptr)) return sh::fail(SH_ERR_INVALID, "%s: NULL buffer", who);
  if (chunks_of(bytes, chunk_bytes) > kMaxChunks)
    return sh::fail(SH_ERR_INVALID, "%s: %llu bytes make more than %llu chunks of %u bytes", who,
                    (unsigned long long)bytes, (unsigned long long)kMaxChunks, chunk_bytes);
  return SH_OK;
}

}  // namespace

namespace sh {

// Launches the comparison for the save-back engine's worker (same checks as sh_block_changed).
int launch_block_changed(const void* buf, uint64_t bytes, uint32_t chunk_bytes, const uint64_t* digests,
                         uint8_t* changed, hipStream_t stream) {
  if (int st = check_args(buf, bytes, chunk_bytes, digests, "sh_block_changed")) return st;
  if (bytes > 0 && changed == nullptr) return sh::fail(SH_ERR_INVALID, "sh_block_changed: changed is NULL");
  if (bytes == 0) return SH_OK;
  const uint64_t n = chunks_of(bytes, chunk_bytes);
  hipLaunchKernelGGL(digest_kernel<true>, dim3((uint32_t)n), dim3(kDigestThreads), 0, stream, (const uint8_t*)buf,
                     bytes, (uint64_t)chunk_bytes, const_cast<uint64_t*>(digests), changed);
  SH_HIP(hipGetLastError());
  return SH_OK;
}

int launch_block_digest(const void* buf, uint64_t bytes, uint32_t chunk_bytes, uint64_t* digests,
                        hipStream_t stream) {
  if (int st = check_args(buf, bytes, chunk_bytes, digests, "sh_block_digest")) return st;
  if (bytes == 0) return SH_OK;
  const uint64_t n = chunks_of(bytes, chunk_bytes);
  hipLaunchKernelGGL(digest_kernel<false>, dim3((uint32_t)n), dim3(kDigestThreads), 0, stream, (const uint8_t*)buf,
                     bytes, (uint64_t)chunk_bytes, digests, (uint8_t*)nullptr);
  SH_HIP(hipGetLastError());
  return SH_OK;
}

}  // namespace sh

extern "C" int sh_block_digest(const void* buf, uint64_t bytes, uint32_t chunk_bytes, uint64_t* digests,
                               void* stream) {
  sh::clear_error();
  return sh::launch_block_digest(buf, bytes, chunk_bytes, digests, (hipStream_t)stream);
}

extern "C" int sh_block_changed(const void* buf, uint64_t bytes, uint32_t chunk_bytes, const uint64_t* digests,
                                uint8_t* changed, void* stream) {
  sh::clear_error();
  return sh::launch_block_changed(buf, bytes, chunk_bytes, digests, changed, (hipStream_t)stream);
}

extern "C" int sh_block_digest_host(const void* buf, uint64_t bytes, uint32_t chunk_bytes, uint64_t* digests) {
  sh::clear_error();
  if (int st = check_args(buf, bytes, chunk_bytes, digests, "sh_block_digest_host")) return st;
  const uint8_t* p = (const uint8_t*)buf;
  const uint64_t n = chunks_of(bytes, chunk_bytes);
  for (uint64_t c = 0; c < n; ++c) {
    const uint64_t b = c * chunk_bytes;
    const uint64_t e = (bytes - b > chunk_bytes) ? b + chunk_bytes : bytes;
    uint64_t sa = 0, sb = 0, off = b;
    for (; off + 16 <= e; off += 16) {
      uint64_t w[2];
      std::memcpy(w, p + off, 16);
      add_word(w[0], off >> 3, sa, sb);
      add_word(w[1], (off >> 3) + 1, sa, sb);
    }
    add_tail(p, off, e, sa, sb);
    digests[2 * c] = sa;
    digests[2 * c + 1] = sb;
  }
  return SH_OK;
}
