// Launch shape of the unpack kernels. Shared by the kernels (sh_unpack.hip, built into the
// library's embedded code object) and the host code that plans and launches them
// (sh_unpack.cpp), which must agree on tile sizes to the element.
#pragma once

#include <cstdint>

#include "stagehand_native.h"

namespace {

// Launch shape, chosen by measurement on MI355X over the config-2 slab: a
// chunk or two per thread and many short-lived 512-thread workgroups stream
// best (dequant two chunks of 8 int8 → 16 B of bf16 each per thread; cast one
// chunk of 4 fp32 → 8 B per thread). Persistent grids, deeper per-thread
// unrolling and wider chunks each measured 5-25% slower, and so did giving each
// XCD a contiguous run of tiles (dequant 2%, cast 6%): neighbouring tiles on
// different XCDs stream faster. Non-temporal accesses help on one side only:
// the dequant's bf16 stores (+1-1.6%) and the cast's fp32 loads (+1.9%); the
// other side, or both, measured slower.
#ifndef SH_UNPACK_THREADS
#define SH_UNPACK_THREADS 512
#endif
#ifndef SH_UNROLL_I8
#define SH_UNROLL_I8 2
#endif
#ifndef SH_UNROLL_F32
#define SH_UNROLL_F32 1
#endif
#ifndef SH_CHUNK_I8
#define SH_CHUNK_I8 8
#endif
#ifndef SH_CHUNK_F32
#define SH_CHUNK_F32 4
#endif

constexpr uint32_t kThreads = SH_UNPACK_THREADS;
// Chunks per thread (lane-interleaved: chunk k of every lane of a wavefront is
// one contiguous span). Measured on config 2 (512 threads): int8 chunks of 8
// twice per thread 6.35 TB/s vs one chunk of 16 6.20 and two of 16 5.41; fp32
// chunks of 4 once per thread 6.06 TB/s vs twice 5.70.
constexpr uint32_t kUnrollI8 = SH_UNROLL_I8;
constexpr uint32_t kUnrollF32 = SH_UNROLL_F32;
constexpr uint32_t kChunkI8 = SH_CHUNK_I8;     // int8 elements per thread per chunk
constexpr uint32_t kChunkF32 = SH_CHUNK_F32;   // fp32 elements per thread per chunk (cast)
constexpr uint32_t kChunkB16 = 16;             // bf16 elements per thread per chunk (widen)
// Byte kinds, per thread per chunk (measured on a 4 GiB region: copy 16 B
// 6.57 TB/s vs 32 B 5.90 and 64 B 5.30; zero fill 32 B 6.29 TB/s vs 16 B 5.08
// and 64 B 5.76).
#ifndef SH_CHUNK_COPY
#define SH_CHUNK_COPY 16
#endif
#ifndef SH_CHUNK_ZERO
#define SH_CHUNK_ZERO 32
#endif
constexpr uint32_t kChunkCopy = SH_CHUNK_COPY;
constexpr uint32_t kChunkZero = SH_CHUNK_ZERO;
static_assert(kChunkCopy % 16 == 0 && kChunkZero % 16 == 0, "byte chunks are whole 16-byte words");
static_assert(kChunkI8 % 4 == 0 && kChunkF32 % 4 == 0, "chunks are whole 32-bit words");
constexpr uint64_t kMaxDescElems = 1ull << 31;

constexpr uint32_t chunk_of(uint32_t kind) {
  return (kind == SH_KIND_I8_ROWSCALE_BF16 || kind == SH_KIND_I8_ROWSCALE_F32) ? kChunkI8
         : kind == SH_KIND_F32_BF16                                              ? kChunkF32
         : kind == SH_KIND_BF16_F32                                              ? kChunkB16
         : kind == SH_KIND_ZERO_BYTES                                            ? kChunkZero
                                                                                 : kChunkCopy;
}
constexpr uint32_t unroll_of(uint32_t kind) {
  return (kind == SH_KIND_I8_ROWSCALE_BF16 || kind == SH_KIND_I8_ROWSCALE_F32) ? kUnrollI8
         : kind == SH_KIND_F32_BF16                                              ? kUnrollF32
                                                                                 : 1u;
}
constexpr uint32_t tile_of(uint32_t kind) { return kThreads * unroll_of(kind) * chunk_of(kind); }
// Most tiles one plan may hold: a launch of n tiles has n * kThreads work-items, below 2^32.
constexpr uint32_t kMaxTiles = 0xFFFFFFFFu / kThreads;

constexpr uint32_t bit(uint32_t kind) { return 1u << kind; }
constexpr uint32_t kMaskDequantBf16 = bit(SH_KIND_I8_ROWSCALE_BF16);
constexpr uint32_t kMaskCastBf16 = bit(SH_KIND_F32_BF16);
constexpr uint32_t kMaskAll = bit(SH_KIND_I8_ROWSCALE_BF16) | bit(SH_KIND_I8_ROWSCALE_F32) |
                              bit(SH_KIND_F32_BF16) | bit(SH_KIND_BF16_F32) |
                              bit(SH_KIND_COPY_BYTES) | bit(SH_KIND_ZERO_BYTES);

// Descriptors travel to the device as kernel arguments, in chunks: no host buffer has to
// outlive the call and no copy is queued from pageable memory.
constexpr uint32_t kDescChunk = 32;  // 2 KiB of descriptors per launch's arguments
struct DescChunk {
  sh_unpack_desc d[kDescChunk];
  uint32_t first;
  uint32_t count;
};

}  // namespace
