// Internal helpers shared by the native sources: error reporting and the
// division-by-invariant used to map a flat element index to its row.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <functional>
#include <string>
#include <vector>

#include "stagehand_native.h"

namespace sh {

// Records the failure text for sh_last_error() on the calling thread and
// returns `status` so call sites can `return fail(...)`.
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// HIP call wrapper: converts a hipError_t into SH_ERR_HIP with the call text.
#define SH_HIP(call)                                                              \
  do {                                                                            \
    hipError_t sh_e_ = (call);                                                    \
    if (sh_e_ != hipSuccess)                                                      \
      return ::sh::fail(SH_ERR_HIP, "HIP error %d (%s) in %s", (int)sh_e_,       \
                        hipGetErrorString(sh_e_), #call);                         \
  } while (0)

// Live native objects by kind, for sh_shutdown's report. Each object struct holds a
// Live<kind> member, so construction and destruction keep the count.
enum LiveKind : int { kLivePool = 0, kLiveLoader, kLiveSaveback, kLiveTurbo, kLiveVmm, kLiveFile, kLiveKinds };
extern std::atomic<int64_t> g_live[kLiveKinds];
template <int K>
struct Live {
  Live() { g_live[K].fetch_add(1, std::memory_order_relaxed); }
  ~Live() { g_live[K].fetch_sub(1, std::memory_order_relaxed); }
  Live(const Live&) = delete;
  Live& operator=(const Live&) = delete;
};

// Names the calling thread (at most 15 characters shown): every thread the library starts
// is called "sh-<role>", so a process can tell them from the runtime's own threads.
void name_thread(const char* name);

// Runs fn(i) for every i in [0, n) on up to `threads` of the shared host copy
// threads (the calling thread included); returns when all calls are done.
void parallel_for(size_t n, unsigned threads, const std::function<void(size_t)>& fn);

// One unit of host staging work: a memcpy (file == nullptr) or a read of
// `bytes` at `file_off` of `file` into dst.
struct IoPiece {
  uint8_t* dst;
  const uint8_t* src;
  sh_file* file;
  uint64_t file_off;
  uint64_t bytes;
};
// Appends a memcpy cut into pieces of at most 8 MiB.
void append_copy(std::vector<IoPiece>& out, void* dst, const void* src, uint64_t bytes);
// Appends a file read cut at 8 MiB file offsets (pieces stay aligned for O_DIRECT).
void append_read(std::vector<IoPiece>& out, sh_file* f, uint64_t file_off, uint64_t bytes, void* dst);
// Checks that [file_off, file_off + bytes) lies inside the file (SH_ERR_INVALID otherwise).
int check_range(const sh_file* f, uint64_t file_off, uint64_t bytes, const char* who);
// Executes the pieces on up to `threads` copy threads; SH_ERR_IO (with the
// failing file, offset and errno in the last error) when a read fails.
int run_io(const std::vector<IoPiece>& pieces, int threads);
// The buffered descriptor of a file that has no O_DIRECT descriptor, else -1:
// the descriptor on which read-ahead advice is worth giving.
int advice_fd(const sh_file* f);

// The library's kernels (sh_kernels.cpp): loaded per device from the embedded code objects on
// first use, unloaded by sh_shutdown.
enum KernelId : int {
  kKernDequantBf16 = 0,
  kKernDequantBf16Zp,
  kKernCastBf16,
  kKernMixed,
  kKernMixedZp,
  kKernPutDescs,
  kKernFillTileMap,
  kKernDigest,
  kKernDigestCompare,
  kKernelCount
};
// Launches kernel `id` of the current device: a 1-D grid of `grid` workgroups of `block`
// work-items on `stream`; args[i] points to the i-th kernel argument.
int launch_kernel(KernelId id, uint32_t grid, uint32_t block, hipStream_t stream, void** args, const char* who);
// Device address of the unpack code object's `scratch` array on the current device.
int noalloc_scratch(void** ptr, const char* who);
// Waits for each device that has the kernels loaded, then unloads them (sh_shutdown).
int unload_kernels();
// Number of devices with the kernels loaded.
int kernels_loaded();
// Ends sh_unpack_noalloc's per-device ordering state (sh_shutdown, before unload_kernels).
void noalloc_release();

// Most chunks one digest launch may cover: one 256-work-item workgroup per chunk, in a 1-D
// grid that stays under 2^32 work-items.
constexpr uint64_t kMaxDigestChunks = 0xFFFFFFFFull / 256u;

// Chunk digests (sh_digest.cpp): the launches behind sh_block_digest / sh_block_changed, for
// the loader and the save-back engine.
int launch_block_digest(const void* buf, uint64_t bytes, uint32_t chunk_bytes, uint64_t* digests, hipStream_t stream);
int launch_block_changed(const void* buf, uint64_t bytes, uint32_t chunk_bytes, const uint64_t* digests,
                         uint8_t* changed, hipStream_t stream);

// floor(n / d) for every 32-bit n, with magic = ceil(2^64 / d) for d >= 2 and
// magic = 0 for d == 1. The quotient is floor(n * magic / 2^64): with
// magic = 2^64/d + eps (0 <= eps < 1), the error term n*eps/2^64 < 2^-32 <= 1/d
// never carries the fractional part of n/d past the next integer.
__host__ __device__ inline uint64_t udiv_magic(uint32_t d) {
  return d <= 1 ? 0ull : (UINT64_MAX / d) + 1ull;
}

__host__ __device__ inline uint32_t udiv(uint32_t n, uint64_t magic) {
  if (magic == 0) return n;
  const uint64_t lo = (uint64_t)n * (uint32_t)magic;
  const uint64_t hi = (uint64_t)n * (uint32_t)(magic >> 32);
  return (uint32_t)((hi + (lo >> 32)) >> 32);
}

}  // namespace sh
