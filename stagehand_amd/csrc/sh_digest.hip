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
