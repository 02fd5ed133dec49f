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
// zero-padded), with l_j and h_j its low and high 32-bit halves and k_j = j * kKey mod 2^32, of
//   A: f(l_j ^ k_j) + f(h_j ^ k_j) * 2^32    and    B: g(l_j ^ k_j) + g(h_j ^ k_j) * 2^32,
// modulo 2^64. f is the 32-bit finalizer of MurmurHash3 (Appleby); g is "lowbias32" (Wellons,
// hash-prospector), the same xorshift-multiply form with other shifts and odd multipliers. Each
// step of either is a bijection of 32-bit words (an xorshift by at least half the width, a
// multiply by an odd constant), so each word's term in A (two 32-bit mixes side by side) is a
// bijection of the keyed word, and a change of one word changes both sums. Several changed
// words leave a chunk's digest unchanged only if their terms' differences cancel in both sums at
// once, which for two unrelated mixers is a chance of about 2^-128 for random changes; it is a
// checksum, not a bound for structured changes. The sums commute, so the digest does not depend
// on how the words are spread over threads.
//
// 32-bit mixers, not 64-bit ones: the kernel is bound by its vector ALU, and a 64-bit multiply
// is three multiply instructions (v_mad_u64_u32 and two v_mul_lo_u32) against one. Measured on
// MI355X over a 740 MiB block: 64-bit SplitMix64/Murmur3 mixers 0.147-0.151 ms (5.1-5.3 TB/s);
// these 0.139-0.142 ms (5.45-5.58 TB/s), and with non-temporal loads 0.126-0.127 ms (6.1 TB/s).

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>

#include "sh_digest_mix.h"
#include "sh_internal.h"
#include "stagehand_native.h"

namespace {

constexpr uint64_t kMaxChunks = sh::kMaxDigestChunks;
static_assert(kMaxChunks == 0xFFFFFFFFull / kDigestThreads, "one workgroup per chunk, under 2^32 work-items");

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
  const uint8_t* b = (const uint8_t*)buf;
  uint64_t chunk = chunk_bytes;
  void* args[] = {(void*)&b, (void*)&bytes, (void*)&chunk, (void*)&digests, (void*)&changed};
  return launch_kernel(kKernDigestCompare, (uint32_t)chunks_of(bytes, chunk_bytes), kDigestThreads, stream, args,
                       "sh_block_changed");
}

int launch_block_digest(const void* buf, uint64_t bytes, uint32_t chunk_bytes, uint64_t* digests,
                        hipStream_t stream) {
  if (int st = check_args(buf, bytes, chunk_bytes, digests, "sh_block_digest")) return st;
  if (bytes == 0) return SH_OK;
  const uint8_t* b = (const uint8_t*)buf;
  uint64_t chunk = chunk_bytes;
  void* args[] = {(void*)&b, (void*)&bytes, (void*)&chunk, (void*)&digests};
  return launch_kernel(kKernDigest, (uint32_t)chunks_of(bytes, chunk_bytes), kDigestThreads, stream, args,
                       "sh_block_digest");
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
