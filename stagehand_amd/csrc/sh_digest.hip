// Chunk-digest kernels for gfx950 (device code only; the digest's definition, the checks and
// the launches are in sh_digest.cpp). Built into a code object that the library embeds and
// loads with the module API (sh_kernels.cpp).

#include <hip/hip_runtime.h>

#include <cstdint>

#include "sh_digest_mix.h"

namespace {

// One workgroup per chunk. COMPARE: changed[c] = 1 when the chunk's digest differs from
// digests[2c], digests[2c + 1], else 0; otherwise the digest is written there.
template <bool COMPARE>
__device__ __forceinline__ void digest_body(const uint8_t* __restrict__ buf, uint64_t bytes, uint64_t chunk,
                                            uint64_t* __restrict__ digests, uint8_t* __restrict__ changed) {
  const uint64_t c = blockIdx.x;
  const uint64_t b = c * chunk;
  const uint64_t e = (bytes - b > chunk) ? b + chunk : bytes;
  const uint64_t n16 = (e - b) / 16;
  uint64_t sa = 0, sb = 0;
  // The key of a thread's first word advances by a constant each iteration (mod 2^32): added,
  // not multiplied per word.
  constexpr uint32_t kStep = 2u * kDigestThreads * kKey;  // words between a thread's iterations, keyed
  uint32_t k = (uint32_t)((b >> 3) + 2ull * threadIdx.x) * kKey;
  // Non-temporal loads: each byte is read once (measured on MI355X over 740 MiB: 6.12-6.14 TB/s
  // against 5.45-5.56 with plain loads). The buffer may start at any byte: the vector type has
  // byte alignment, and gfx950 runs 16-byte loads at any address in its unaligned-access mode.
  typedef uint32_t u32x4_a1 __attribute__((ext_vector_type(4), aligned(1)));
  const u32x4_a1* p = reinterpret_cast<const u32x4_a1*>(buf + b);
#pragma unroll 4
  for (uint64_t i = threadIdx.x; i < n16; i += kDigestThreads) {
    const u32x4_a1 w = __builtin_nontemporal_load(p + i);
    add_keyed((uint64_t)w.x | ((uint64_t)w.y << 32), k, sa, sb);
    add_keyed((uint64_t)w.z | ((uint64_t)w.w << 32), k + kKey, sa, sb);
    k += kStep;
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

}  // namespace

extern "C" __global__ __launch_bounds__(kDigestThreads) void sh_digest_kernel(const uint8_t* __restrict__ buf,
                                                                              uint64_t bytes, uint64_t chunk,
                                                                              uint64_t* __restrict__ digests) {
  digest_body<false>(buf, bytes, chunk, digests, nullptr);
}

extern "C" __global__ __launch_bounds__(kDigestThreads) void sh_digest_compare_kernel(
    const uint8_t* __restrict__ buf, uint64_t bytes, uint64_t chunk, const uint64_t* __restrict__ digests,
    uint8_t* __restrict__ changed) {
  digest_body<true>(buf, bytes, chunk, const_cast<uint64_t*>(digests), changed);
}
