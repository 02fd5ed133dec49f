// Slab unpack kernels for gfx950: SquareQ INT8→bf16 dequant and fp32→bf16
// cast, scattering a packed device-resident source slab into a block's
// contiguous parameter buffer.
//
// Replaces the host-side staging arithmetic of the reference:
//   SquareQ dequant   src/stagehand/scheduler.py:290-300
//   bias / param cast src/stagehand/scheduler.py:181, 224-230, 302-306, 1066-1071
//   zero-fill         src/stagehand/scheduler.py:240, 276-297, 325
//
// Work decomposition. Every descriptor covers rows*cols elements, cut into
// tiles of kThreads * unroll * chunk elements; a host-built tile map gives
// each workgroup its descriptor in O(1) (one scalar load), and the descriptor
// itself is a 64-byte scalar load, so all per-region state lives in SGPRs.
// Each thread moves `unroll` chunks; all loads of a thread are issued before
// the first conversion. Loads and stores are up to 128-bit (an int8 chunk of
// 8 is a 64-bit load and a 128-bit bf16 store; the cast reads 128 and writes
// 64 bits); the hardware's unaligned-access mode lets them start at any byte
// offset, which the reference layout needs (it has no padding, so int8 regions
// start at arbitrary offsets). With int8 chunks of 8, every chunk of a row
// whose length is a multiple of 8 needs one row scale, loaded once per chunk;
// shorter or ragged rows take an element-wise path. This is pure
// streaming: no LDS (the scale is one load per chunk) and no MFMA.
//
// Numerics. The dequant is computed exactly as the reference's torch CPU ops:
// f32(q) exactly, then an IEEE fp32 subtract of the zero point (skipped when
// no zero points are given: q - 0.0f == q bit for bit), then an IEEE fp32
// multiply by the row scale, each rounded to nearest even; fp32 denormals are
// kept (no flush flags). Contraction is disabled so nothing becomes an FMA.
// fp32→bf16 is round-to-nearest-even on the bit pattern,
//   bf16 = (u + 0x7FFF + ((u >> 16) & 1)) >> 16,
// which equals torch's CPU conversion for every non-NaN input; every NaN
// becomes 0xFFFF, as torch's CPU conversion does.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <new>
#include <mutex>
#include <vector>

#include "sh_internal.h"
#include "stagehand_native.h"

#pragma clang fp contract(off)

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

// NB bytes as 32-bit words; loaded and stored with unaligned-capable 128-bit
// (or 64-bit) vector memory operations.
template <uint32_t NB>
struct Words {
  uint32_t w[NB / 4];
};

template <uint32_t NB>
__device__ __forceinline__ Words<NB> ldw(const uint8_t* p) {
  Words<NB> v;
  __builtin_memcpy(&v, p, NB);
  return v;
}

template <uint32_t NB>
__device__ __forceinline__ void stw(uint8_t* p, const Words<NB>& v) {
  __builtin_memcpy(p, &v, NB);
}

// Non-temporal forms (the `nt` bit on the load / store): 8 or 16 bytes, any byte alignment.
typedef uint32_t u32x2_a1 __attribute__((ext_vector_type(2), aligned(1)));
typedef uint32_t u32x4_a1 __attribute__((ext_vector_type(4), aligned(1)));

template <uint32_t NB>
__device__ __forceinline__ Words<NB> ldw_nt(const uint8_t* p) {
  static_assert(NB == 8 || NB == 16, "8- or 16-byte non-temporal loads");
  Words<NB> v;
  if constexpr (NB == 8) {
    const u32x2_a1 x = __builtin_nontemporal_load(reinterpret_cast<const u32x2_a1*>(p));
    v.w[0] = x.x;
    v.w[1] = x.y;
  } else {
    const u32x4_a1 x = __builtin_nontemporal_load(reinterpret_cast<const u32x4_a1*>(p));
    v.w[0] = x.x;
    v.w[1] = x.y;
    v.w[2] = x.z;
    v.w[3] = x.w;
  }
  return v;
}

template <uint32_t NB>
__device__ __forceinline__ void stw_nt(uint8_t* p, const Words<NB>& v) {
  static_assert(NB == 8 || NB == 16, "8- or 16-byte non-temporal stores");
  if constexpr (NB == 8) {
    u32x2_a1 x;
    x.x = v.w[0];
    x.y = v.w[1];
    __builtin_nontemporal_store(x, reinterpret_cast<u32x2_a1*>(p));
  } else {
    u32x4_a1 x;
    x.x = v.w[0];
    x.y = v.w[1];
    x.z = v.w[2];
    x.w = v.w[3];
    __builtin_nontemporal_store(x, reinterpret_cast<u32x4_a1*>(p));
  }
}

// Rounded bf16 in bits 31..16 (low half is garbage): u + 0x7FFF + lsb.
__device__ __forceinline__ uint32_t rne_hi(float x) {
  const uint32_t u = __float_as_uint(x);
  return u + 0x7FFFu + ((u >> 16) & 1u);
}

__device__ __forceinline__ uint32_t rne_hi_nan(float x) {
  return (x != x) ? 0xFFFFFFFFu : rne_hi(x);
}

// Packs the upper halves of two rne_hi words: lo element in bits 15..0.
__device__ __forceinline__ uint32_t pack_hi(uint32_t lo, uint32_t hi) {
  return __builtin_amdgcn_perm(hi, lo, 0x07060302u);
}

__device__ __forceinline__ uint16_t bf16_bits(float x) { return (uint16_t)(rne_hi_nan(x) >> 16); }

__device__ __forceinline__ float i8_at(uint32_t word, uint32_t byte) {
  return (float)(int32_t)(int8_t)(uint8_t)(word >> (8 * byte));
}

template <bool HAS_ZP>
__device__ __forceinline__ float dq(float q, float s, float z) {
  if (HAS_ZP) q = q - z;
  return q * s;
}

// ── INT8 row-scale dequant ────────────────────────────────────────────────

// One chunk of C int8 values of a single row → C outputs.
template <uint32_t C, bool OUT_BF16, bool HAS_ZP, bool NANCHK>
__device__ __forceinline__ void dq_chunk_store(const Words<C>& q, float s, float z, uint8_t* out) {
  if (OUT_BF16) {
    Words<2 * C> o;
#pragma unroll
    for (uint32_t w = 0; w < C / 4; ++w) {
      const uint32_t word = q.w[w];
      const float f0 = dq<HAS_ZP>(i8_at(word, 0), s, z);
      const float f1 = dq<HAS_ZP>(i8_at(word, 1), s, z);
      const float f2 = dq<HAS_ZP>(i8_at(word, 2), s, z);
      const float f3 = dq<HAS_ZP>(i8_at(word, 3), s, z);
      o.w[2 * w] = NANCHK ? pack_hi(rne_hi_nan(f0), rne_hi_nan(f1)) : pack_hi(rne_hi(f0), rne_hi(f1));
      o.w[2 * w + 1] = NANCHK ? pack_hi(rne_hi_nan(f2), rne_hi_nan(f3)) : pack_hi(rne_hi(f2), rne_hi(f3));
    }
    stw_nt<2 * C>(out, o);  // written once, read by the next kernel: no reason to keep it in L2
  } else {
    Words<4 * C> o;
#pragma unroll
    for (uint32_t j = 0; j < C; ++j) o.w[j] = __float_as_uint(dq<HAS_ZP>(i8_at(q.w[j / 4], j % 4), s, z));
    stw<4 * C>(out, o);
  }
}

template <bool OUT_BF16>
__device__ __forceinline__ void store_elem(uint8_t* o, uint32_t idx, float v) {
  if (OUT_BF16) {
    const uint16_t b = bf16_bits(v);
    __builtin_memcpy(o + 2 * (size_t)idx, &b, 2);
  } else {
    __builtin_memcpy(o + 4 * (size_t)idx, &v, 4);
  }
}

template <bool OUT_BF16, bool HAS_ZP>
__device__ __forceinline__ void tile_i8(const sh_unpack_desc& d, uint32_t local,
                                        const uint8_t* __restrict__ src,
                                        const float* __restrict__ scales,
                                        const float* __restrict__ zps, uint8_t* __restrict__ dst) {
  constexpr uint32_t C = kChunkI8;
  constexpr uint32_t U = kUnrollI8;
  constexpr uint32_t kOutBytes = OUT_BF16 ? 2 : 4;
  const uint32_t cols = d.cols;
  const uint32_t numel = d.rows * cols;
  const uint32_t ld = d.src_ld ? d.src_ld : cols;
  const uint8_t* s = src + d.src_off;
  uint8_t* o = dst + d.dst_off;
  const float* sc = scales + d.scale_off;
  const float* zp = HAS_ZP ? zps + d.scale_off : nullptr;
  // d.lead elements precede element 0 in the first tile; a chunk before the region wraps to an
  // index >= 2^32 - 64, above every numel, and is skipped by the bounds checks below
  const uint32_t e0 = local * (kThreads * U * C) + threadIdx.x * C - d.lead;

  if (ld == cols && (cols % C) == 0) {
    // Every chunk lies inside one row: one scale per chunk.
    Words<C> q[U];
    float sv[U], zv[U];
#pragma unroll
    for (uint32_t k = 0; k < U; ++k) {
      const uint32_t e = e0 + k * (kThreads * C);
      if (e < numel) q[k] = ldw<C>(s + e);
    }
#pragma unroll
    for (uint32_t k = 0; k < U; ++k) {
      const uint32_t e = e0 + k * (kThreads * C);
      if (e < numel) {
        const uint32_t r = sh::udiv(e, d.div_magic);
        sv[k] = sc[r];
        zv[k] = HAS_ZP ? zp[r] : 0.0f;
      }
    }
#pragma unroll
    for (uint32_t k = 0; k < U; ++k) {
      const uint32_t e = e0 + k * (kThreads * C);
      if (e < numel) {
        uint8_t* out = o + (size_t)e * kOutBytes;
        // A finite scale and zero point cannot turn a finite q into NaN.
        if (__builtin_isfinite(sv[k]) && (!HAS_ZP || __builtin_isfinite(zv[k])))
          dq_chunk_store<C, OUT_BF16, HAS_ZP, false>(q[k], sv[k], zv[k], out);
        else
          dq_chunk_store<C, OUT_BF16, HAS_ZP, true>(q[k], sv[k], zv[k], out);
      }
    }
    return;
  }

  // Rows that are not a multiple of the chunk, or a padded source (ld > cols):
  // element-wise, with the row tracked incrementally inside each chunk.
#pragma unroll 1
  for (uint32_t k = 0; k < U; ++k) {
    const uint32_t e = e0 + k * (kThreads * C);
    if (e >= numel) continue;
    uint32_t r = sh::udiv(e, d.div_magic);
    uint32_t c = e - r * cols;
    const uint32_t n = min(C, numel - e);
    if (ld == cols && n == C) {
      const Words<C> q = ldw<C>(s + e);
      if (OUT_BF16) {
        uint32_t hw[C];
#pragma unroll
        for (uint32_t j = 0; j < C; ++j) {
          hw[j] = rne_hi_nan(dq<HAS_ZP>(i8_at(q.w[j / 4], j % 4), sc[r], HAS_ZP ? zp[r] : 0.0f));
          if (++c == cols) {
            c = 0;
            ++r;
          }
        }
        Words<2 * C> ow;
#pragma unroll
        for (uint32_t w = 0; w < C / 2; ++w) ow.w[w] = pack_hi(hw[2 * w], hw[2 * w + 1]);
        stw<2 * C>(o + (size_t)e * 2, ow);
      } else {
        Words<4 * C> ow;
#pragma unroll
        for (uint32_t j = 0; j < C; ++j) {
          ow.w[j] = __float_as_uint(dq<HAS_ZP>(i8_at(q.w[j / 4], j % 4), sc[r], HAS_ZP ? zp[r] : 0.0f));
          if (++c == cols) {
            c = 0;
            ++r;
          }
        }
        stw<4 * C>(o + (size_t)e * 4, ow);
      }
    } else {
      for (uint32_t j = 0; j < n; ++j) {
        const float q = (float)(int32_t)(int8_t)s[(size_t)r * ld + c];
        store_elem<OUT_BF16>(o, e + j, dq<HAS_ZP>(q, sc[r], HAS_ZP ? zp[r] : 0.0f));
        if (++c == cols) {
          c = 0;
          ++r;
        }
      }
    }
  }
}

// ── fp32 → bf16 cast ──────────────────────────────────────────────────────

__device__ __forceinline__ void tile_f32_bf16(const sh_unpack_desc& d, uint32_t local,
                                              const uint8_t* __restrict__ src,
                                              uint8_t* __restrict__ dst) {
  constexpr uint32_t C = kChunkF32;
  constexpr uint32_t U = kUnrollF32;
  const uint32_t numel = d.rows * d.cols;
  const uint8_t* s = src + d.src_off;
  uint8_t* o = dst + d.dst_off;
  const uint32_t e0 = local * (kThreads * U * C) + threadIdx.x * C - d.lead;  // wraps before the region
  Words<4 * C> v[U];
#pragma unroll
  for (uint32_t k = 0; k < U; ++k) {
    const uint32_t e = e0 + k * (kThreads * C);
    if (e < numel && numel - e >= C) v[k] = ldw_nt<4 * C>(s + (size_t)e * 4);  // read once
  }
#pragma unroll
  for (uint32_t k = 0; k < U; ++k) {
    const uint32_t e = e0 + k * (kThreads * C);
    if (e < numel && numel - e >= C) {
      Words<2 * C> ow;
#pragma unroll
      for (uint32_t w = 0; w < C / 2; ++w)
        ow.w[w] = pack_hi(rne_hi_nan(__uint_as_float(v[k].w[2 * w])), rne_hi_nan(__uint_as_float(v[k].w[2 * w + 1])));
      stw<2 * C>(o + (size_t)e * 2, ow);
    } else if (e < numel) {
      for (uint32_t j = e; j < numel; ++j) {
        float x;
        __builtin_memcpy(&x, s + (size_t)j * 4, 4);
        const uint16_t b = bf16_bits(x);
        __builtin_memcpy(o + (size_t)j * 2, &b, 2);
      }
    }
  }
}

// ── bf16 → fp32 widen ─────────────────────────────────────────────────────

__device__ __forceinline__ void tile_bf16_f32(const sh_unpack_desc& d, uint32_t local,
                                              const uint8_t* __restrict__ src,
                                              uint8_t* __restrict__ dst) {
  constexpr uint32_t C = kChunkB16;
  constexpr uint32_t U = 1;
  const uint32_t numel = d.rows * d.cols;
  const uint8_t* s = src + d.src_off;
  uint8_t* o = dst + d.dst_off;
  const uint32_t e0 = local * (kThreads * U * C) + threadIdx.x * C - d.lead;  // wraps before the region
  Words<2 * C> v[U];
#pragma unroll
  for (uint32_t k = 0; k < U; ++k) {
    const uint32_t e = e0 + k * (kThreads * C);
    if (e < numel && numel - e >= C) v[k] = ldw<2 * C>(s + (size_t)e * 2);
  }
#pragma unroll
  for (uint32_t k = 0; k < U; ++k) {
    const uint32_t e = e0 + k * (kThreads * C);
    if (e < numel && numel - e >= C) {
      Words<4 * C> ow;
#pragma unroll
      for (uint32_t w = 0; w < C / 2; ++w) {
        ow.w[2 * w] = v[k].w[w] << 16;
        ow.w[2 * w + 1] = v[k].w[w] & 0xFFFF0000u;
      }
      stw<4 * C>(o + (size_t)e * 4, ow);
    } else if (e < numel) {
      for (uint32_t j = e; j < numel; ++j) {
        uint16_t b;
        __builtin_memcpy(&b, s + (size_t)j * 2, 2);
        const uint32_t w = (uint32_t)b << 16;
        __builtin_memcpy(o + (size_t)j * 4, &w, 4);
      }
    }
  }
}

// ── byte copy / zero fill ─────────────────────────────────────────────────

template <bool ZERO>
__device__ __forceinline__ void tile_bytes(const sh_unpack_desc& d, uint32_t local,
                                           const uint8_t* __restrict__ src,
                                           uint8_t* __restrict__ dst) {
  // A tile is kThreads * U * C bytes, moved as 16-byte words with
  // consecutive lanes on consecutive words (each load / store instruction of a
  // wavefront covers one contiguous 1 KiB span).
  constexpr uint32_t C = ZERO ? kChunkZero : kChunkCopy;
  constexpr uint32_t U = 1;
  constexpr uint32_t W = 16;
  constexpr uint32_t kWords = U * (C / W);
  const uint32_t nbytes = d.rows * d.cols;
  const uint8_t* s = src + d.src_off;
  uint8_t* o = dst + d.dst_off;
  const uint32_t t0 = local * (kThreads * U * C) - d.lead;  // wraps before the region
  Words<W> v[kWords];
#pragma unroll
  for (uint32_t k = 0; k < kWords; ++k) {
    const uint32_t b = t0 + (k * kThreads + threadIdx.x) * W;
    if (b < nbytes && nbytes - b >= W) {
      if (ZERO) {
#pragma unroll
        for (uint32_t w = 0; w < W / 4; ++w) v[k].w[w] = 0;
      } else {
        v[k] = ldw<W>(s + b);
      }
    }
  }
#pragma unroll
  for (uint32_t k = 0; k < kWords; ++k) {
    const uint32_t b = t0 + (k * kThreads + threadIdx.x) * W;
    if (b < nbytes && nbytes - b >= W) {
      stw<W>(o + b, v[k]);
    } else if (b < nbytes) {
      for (uint32_t j = b; j < nbytes; ++j) o[j] = ZERO ? (uint8_t)0 : s[j];
    }
  }
}

// ── kernels ───────────────────────────────────────────────────────────────

constexpr uint32_t bit(uint32_t kind) { return 1u << kind; }
constexpr uint32_t kMaskDequantBf16 = bit(SH_KIND_I8_ROWSCALE_BF16);
constexpr uint32_t kMaskCastBf16 = bit(SH_KIND_F32_BF16);
constexpr uint32_t kMaskAll = bit(SH_KIND_I8_ROWSCALE_BF16) | bit(SH_KIND_I8_ROWSCALE_F32) |
                              bit(SH_KIND_F32_BF16) | bit(SH_KIND_BF16_F32) |
                              bit(SH_KIND_COPY_BYTES) | bit(SH_KIND_ZERO_BYTES);

// Reads a whole descriptor before any of its fields is tested. Left to itself the compiler
// loads the kind, branches on it and only then loads the fields the branch uses: one more round
// of dependent scalar loads at the start of every workgroup (tile map entry, kind, fields).
__device__ __forceinline__ sh_unpack_desc load_desc(const sh_unpack_desc* __restrict__ p) {
  static_assert(sizeof(sh_unpack_desc) == 64, "descriptor is 16 dwords");
  uint32_t w[16];
  __builtin_memcpy(w, p, sizeof w);
#pragma unroll
  for (int i = 0; i < 16; ++i) asm volatile("" : "+s"(w[i]));  // every dword in an SGPR here
  sh_unpack_desc d;
  __builtin_memcpy(&d, w, sizeof d);
  return d;
}

template <uint32_t MASK, bool HAS_ZP>
__device__ __forceinline__ void unpack_body(const sh_unpack_desc* __restrict__ descs,
                                            const uint32_t* __restrict__ tile_map,
                                            const uint8_t* __restrict__ src,
                                            const float* __restrict__ scales,
                                            const float* __restrict__ zps,
                                            uint8_t* __restrict__ dst) {
  const uint32_t tile = blockIdx.x;
  const sh_unpack_desc d = load_desc(descs + tile_map[tile]);
  const uint32_t local = tile - d.tile_begin;
  // The single-kind kernels are launched only for plans whose every descriptor has that kind
  // (launch_tiles), so they test no kind.
  if constexpr (MASK == kMaskDequantBf16) {
    tile_i8<true, HAS_ZP>(d, local, src, scales, zps, dst);
    return;
  }
  if constexpr (MASK == kMaskCastBf16) {
    tile_f32_bf16(d, local, src, dst);
    return;
  }
  switch (d.kind) {
    case SH_KIND_I8_ROWSCALE_BF16:
      if constexpr ((MASK & bit(SH_KIND_I8_ROWSCALE_BF16)) != 0)
        tile_i8<true, HAS_ZP>(d, local, src, scales, zps, dst);
      break;
    case SH_KIND_I8_ROWSCALE_F32:
      if constexpr ((MASK & bit(SH_KIND_I8_ROWSCALE_F32)) != 0)
        tile_i8<false, HAS_ZP>(d, local, src, scales, zps, dst);
      break;
    case SH_KIND_F32_BF16:
      if constexpr ((MASK & bit(SH_KIND_F32_BF16)) != 0) tile_f32_bf16(d, local, src, dst);
      break;
    case SH_KIND_BF16_F32:
      if constexpr ((MASK & bit(SH_KIND_BF16_F32)) != 0) tile_bf16_f32(d, local, src, dst);
      break;
    case SH_KIND_COPY_BYTES:
      if constexpr ((MASK & bit(SH_KIND_COPY_BYTES)) != 0) tile_bytes<false>(d, local, src, dst);
      break;
    case SH_KIND_ZERO_BYTES:
      if constexpr ((MASK & bit(SH_KIND_ZERO_BYTES)) != 0) tile_bytes<true>(d, local, src, dst);
      break;
    default:
      break;
  }
}

}  // namespace

#define SH_KERNEL_ARGS                                                                 \
  const sh_unpack_desc *__restrict__ descs, const uint32_t *__restrict__ tile_map,    \
      const uint8_t *__restrict__ src, const float *__restrict__ scales,              \
      const float *__restrict__ zps, uint8_t *__restrict__ dst

extern "C" __global__ __launch_bounds__(kThreads) void sh_dequant_i8_bf16_kernel(SH_KERNEL_ARGS) {
  unpack_body<kMaskDequantBf16, false>(descs, tile_map, src, scales, zps, dst);
}
extern "C" __global__ __launch_bounds__(kThreads) void sh_dequant_i8_bf16_zp_kernel(SH_KERNEL_ARGS) {
  unpack_body<kMaskDequantBf16, true>(descs, tile_map, src, scales, zps, dst);
}
extern "C" __global__ __launch_bounds__(kThreads) void sh_cast_f32_bf16_kernel(SH_KERNEL_ARGS) {
  unpack_body<kMaskCastBf16, false>(descs, tile_map, src, scales, zps, dst);
}
extern "C" __global__ __launch_bounds__(kThreads) void sh_unpack_mixed_kernel(SH_KERNEL_ARGS) {
  unpack_body<kMaskAll, false>(descs, tile_map, src, scales, zps, dst);
}
extern "C" __global__ __launch_bounds__(kThreads) void sh_unpack_mixed_zp_kernel(SH_KERNEL_ARGS) {
  unpack_body<kMaskAll, true>(descs, tile_map, src, scales, zps, dst);
}

// ── allocation-free launches (sh_unpack_noalloc) ─────────────────────────────
//
// The launch table and the tile map of a call live in this file-scope array, one copy per
// GPU, held until the process ends: descriptors at offset 0, the tile map after them. In
// host code `scratch` is only a stand-in for the symbol; the device address comes from
// hipGetSymbolAddress (scratch_on_current_device below).
static_assert(SH_UNPACK_NOALLOC_SCRATCH_BYTES ==
                  SH_UNPACK_NOALLOC_MAX_DESCS * sizeof(sh_unpack_desc) + SH_UNPACK_NOALLOC_MAX_TILES * 4ull,
              "scratch layout: descriptor table, then one uint32 per tile");
static __device__ __align__(256) uint8_t scratch[SH_UNPACK_NOALLOC_SCRATCH_BYTES];

// Descriptors travel to the device as kernel arguments, in chunks: no host buffer has to
// outlive the call and no copy is queued from pageable memory.
constexpr uint32_t kDescChunk = 32;  // 2 KiB of descriptors per launch's arguments
struct DescChunk {
  sh_unpack_desc d[kDescChunk];
  uint32_t first;
  uint32_t count;
};

extern "C" __global__ __launch_bounds__(kDescChunk) void sh_put_descs_kernel(DescChunk c, sh_unpack_desc* table) {
  if (threadIdx.x < c.count) table[c.first + threadIdx.x] = c.d[threadIdx.x];
}

// map[t] = the descriptor whose tiles [tile_begin, tile_begin + ntiles) hold t. Descriptors
// hold consecutive, non-empty tile ranges in table order, so a binary search over tile_begin
// finds it.
extern "C" __global__ __launch_bounds__(256) void sh_fill_tile_map_kernel(const sh_unpack_desc* __restrict__ table,
                                                                          uint32_t n, uint32_t* __restrict__ map,
                                                                          uint32_t n_tiles) {
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  if (t >= n_tiles) return;
  uint32_t lo = 0, hi = n - 1;
  while (lo < hi) {
    const uint32_t mid = (lo + hi + 1) >> 1;
    if (table[mid].tile_begin <= t) lo = mid;
    else hi = mid - 1;
  }
  map[t] = lo;
}

namespace {

// ── host side: plans ──────────────────────────────────────────────────────

bool is_i8(uint32_t kind) {
  return kind == SH_KIND_I8_ROWSCALE_BF16 || kind == SH_KIND_I8_ROWSCALE_F32;
}
bool is_bytes(uint32_t kind) { return kind == SH_KIND_COPY_BYTES || kind == SH_KIND_ZERO_BYTES; }
uint32_t src_elem_bytes(uint32_t kind) {
  switch (kind) {
    case SH_KIND_I8_ROWSCALE_BF16:
    case SH_KIND_I8_ROWSCALE_F32:
    case SH_KIND_COPY_BYTES: return 1;
    case SH_KIND_F32_BF16: return 4;
    case SH_KIND_BF16_F32: return 2;
    default: return 0;  // ZERO reads nothing
  }
}
uint32_t dst_elem_bytes(uint32_t kind) {
  switch (kind) {
    case SH_KIND_I8_ROWSCALE_BF16:
    case SH_KIND_F32_BF16: return 2;
    case SH_KIND_I8_ROWSCALE_F32:
    case SH_KIND_BF16_F32: return 4;
    default: return 1;
  }
}

// Elements placed before element 0 in a descriptor's first tile, so that the tiles' destination
// spans start on kDstAlign-byte boundaries of the destination buffer (whose base the caller's
// allocator aligns to at least that), or failing that on 64-byte lines. Measured on MI355X:
// - a region that starts inside a 64-byte line has every wavefront write a partial line at both
//   ends, shared with the neighbouring wavefront, often on another XCD; a 2.2 G-element dequant
//   region whose destination started 16 or 32 bytes into a line ran 1.9% slower, a cast 1.2%;
// - line-aligned tiles still lose to tiles on 1 KiB or larger boundaries: a flat cast whose
//   destination tiles started 512 B past a 1 KiB boundary ran 1.3% slower, at 64 B past one
//   8.8%; on the config-2 slab, 4 KiB against 64-byte alignment raised the dequant from 6.44-6.48
//   to 6.55-6.57 TB/s and the cast from 6.19-6.21 to 6.26-6.28.
// The lead is below one tile for every kind (at most 4095 destination bytes), so a region gains
// at most one tile. It keeps chunks in their place relative to the region (a multiple of the
// chunk), so a region whose start allows no such lead gets none. 64 bytes of destination are a
// whole number of chunks for every kind, so a region that could be put on a 64-byte line can be
// put on a kDstAlign boundary.
constexpr uint64_t kDstAlign = 4096;
uint32_t lead_of(uint32_t kind, uint64_t dst_off) {
  const uint64_t ob = dst_elem_bytes(kind);
  const uint64_t mis = dst_off % kDstAlign;
  if (mis == 0 || mis % ob != 0) return 0;
  const uint64_t lead = mis / ob;
  return lead % chunk_of(kind) == 0 ? (uint32_t)lead : 0u;
}

}  // namespace

struct sh_plan {
  int device = -1;
  std::vector<sh_unpack_desc> host;
  sh_unpack_desc* d_descs = nullptr;
  uint32_t* d_tile_map = nullptr;
  sh_plan_info info{};
};

namespace {

// Validates the caller's descriptors and produces the launch table (oversize
// regions split, tiles assigned) and its summary. Host only: no device calls.
int build_table(const sh_unpack_desc* descs, uint32_t n, std::vector<sh_unpack_desc>& table,
                sh_plan_info& info, const char* who) {
  if (n > 0 && descs == nullptr) return sh::fail(SH_ERR_INVALID, "%s: descs is NULL", who);
  table.clear();
  table.reserve(n);
  info = sh_plan_info{};
  info.tile_elems = tile_of(SH_KIND_I8_ROWSCALE_BF16);
  uint64_t tiles = 0;

  auto push = [&](sh_unpack_desc d) -> int {
    const uint64_t numel = (uint64_t)d.rows * d.cols;
    d.div_magic = sh::udiv_magic(d.cols);
    d.lead = lead_of(d.kind, d.dst_off);
    const uint64_t per_tile = tile_of(d.kind);
    const uint64_t nt = (numel + d.lead + per_tile - 1) / per_tile;
    // one workgroup of kThreads work-items per tile, in a 1-D grid: the launch must stay
    // under 2^32 work-items
    if (tiles + nt > kMaxTiles)
      return sh::fail(SH_ERR_INVALID, "%s: plan needs more than %u tiles (%u work-items each); split it",
                      who, kMaxTiles, kThreads);
    d.tile_begin = (uint32_t)tiles;
    d.ntiles = (uint32_t)nt;
    d.reserved = 0;
    tiles += nt;
    const uint32_t ld = d.src_ld ? d.src_ld : d.cols;
    const uint64_t src_span =
        is_i8(d.kind) ? ((uint64_t)(d.rows - 1) * ld + d.cols) : numel * src_elem_bytes(d.kind);
    if (d.kind != SH_KIND_ZERO_BYTES) info.src_extent = std::max(info.src_extent, d.src_off + src_span);
    info.dst_extent = std::max(info.dst_extent, d.dst_off + numel * dst_elem_bytes(d.kind));
    if (is_i8(d.kind)) {
      info.scale_extent = std::max(info.scale_extent, d.scale_off + d.rows);
      info.algo_bytes += 4ull * d.rows;
    }
    info.algo_bytes += numel * (src_elem_bytes(d.kind) + dst_elem_bytes(d.kind));
    info.elements += numel;
    info.kind_mask |= bit(d.kind);
    table.push_back(d);
    return SH_OK;
  };

  for (uint32_t i = 0; i < n; ++i) {
    sh_unpack_desc d = descs[i];
    if (d.kind < SH_KIND_I8_ROWSCALE_BF16 || d.kind > SH_KIND_ZERO_BYTES)
      return sh::fail(SH_ERR_INVALID, "%s: descriptor %u has unknown kind %u", who, i, d.kind);
    if (d.rows == 0 || d.cols == 0) continue;  // empty region: nothing to write
    const uint32_t ld = d.src_ld ? d.src_ld : d.cols;
    if (is_i8(d.kind)) {
      if (ld < d.cols)
        return sh::fail(SH_ERR_INVALID, "%s: descriptor %u has src_ld %u < cols %u", who, i, ld, d.cols);
      if (d.cols > kMaxDescElems)
        return sh::fail(SH_ERR_INVALID, "%s: descriptor %u row of %u elements is too long", who, i, d.cols);
      d.src_ld = ld;
      // Split by rows so every piece holds at most 2^31 elements (32-bit indexing in the kernel).
      const uint32_t rows_per = (uint32_t)std::min<uint64_t>(d.rows, kMaxDescElems / d.cols);
      for (uint32_t r0 = 0; r0 < d.rows; r0 += rows_per) {
        sh_unpack_desc p = d;
        p.rows = std::min(rows_per, d.rows - r0);
        p.src_off = d.src_off + (uint64_t)r0 * ld;
        p.dst_off = d.dst_off + (uint64_t)r0 * d.cols * dst_elem_bytes(d.kind);
        p.scale_off = d.scale_off + r0;
        if (int st = push(p)) return st;
      }
    } else {
      if (ld != d.cols)
        return sh::fail(SH_ERR_INVALID, "%s: descriptor %u of kind %u must be contiguous (src_ld == cols)", who, i, d.kind);
      // Flat region: re-cut into rows of at most 2^30 elements.
      uint64_t numel = (uint64_t)d.rows * d.cols;
      uint64_t done = 0;
      while (done < numel) {
        const uint64_t piece = std::min<uint64_t>(numel - done, 1ull << 30);
        sh_unpack_desc p = d;
        p.rows = 1;
        p.cols = (uint32_t)piece;
        p.src_ld = (uint32_t)piece;
        p.src_off = d.src_off + done * src_elem_bytes(d.kind);
        p.dst_off = d.dst_off + done * dst_elem_bytes(d.kind);
        if (int st = push(p)) return st;
        done += piece;
      }
    }
  }
  info.n_desc = (uint32_t)table.size();
  info.n_tiles = (uint32_t)tiles;
  return SH_OK;
}

}  // namespace

extern "C" int sh_plan_describe(const sh_unpack_desc* descs, uint32_t n, sh_plan_info* info) {
  sh::clear_error();
  if (info == nullptr) return sh::fail(SH_ERR_INVALID, "sh_plan_describe: info is NULL");
  std::vector<sh_unpack_desc> table;
  return build_table(descs, n, table, *info, "sh_plan_describe");
}

extern "C" int sh_plan_create(const sh_unpack_desc* descs, uint32_t n, sh_plan** out) {
  sh::clear_error();
  if (out == nullptr) return sh::fail(SH_ERR_INVALID, "sh_plan_create: out is NULL");
  *out = nullptr;
  std::vector<sh_unpack_desc> table;
  sh_plan_info info{};
  if (int st = build_table(descs, n, table, info, "sh_plan_create")) return st;
  const uint64_t tiles = info.n_tiles;

  sh_plan* plan = new (std::nothrow) sh_plan();
  if (plan == nullptr) return sh::fail(SH_ERR_OOM, "sh_plan_create: out of host memory");
  plan->host = std::move(table);
  plan->info = info;
  hipError_t e = hipGetDevice(&plan->device);
  if (e != hipSuccess) {
    delete plan;
    return sh::fail(SH_ERR_HIP, "HIP error %d (%s) in hipGetDevice", (int)e, hipGetErrorString(e));
  }
  if (!plan->host.empty()) {
    std::vector<uint32_t> tile_map(tiles);
    for (uint32_t i = 0; i < plan->host.size(); ++i) {
      const sh_unpack_desc& d = plan->host[i];
      std::fill(tile_map.begin() + d.tile_begin, tile_map.begin() + d.tile_begin + d.ntiles, i);
    }
    const size_t desc_bytes = plan->host.size() * sizeof(sh_unpack_desc);
    const size_t map_bytes = tile_map.size() * sizeof(uint32_t);
    e = hipMalloc((void**)&plan->d_descs, desc_bytes);
    if (e == hipSuccess) e = hipMalloc((void**)&plan->d_tile_map, map_bytes);
    if (e == hipSuccess) e = hipMemcpy(plan->d_descs, plan->host.data(), desc_bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(plan->d_tile_map, tile_map.data(), map_bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      (void)hipFree(plan->d_descs);
      (void)hipFree(plan->d_tile_map);
      delete plan;
      return sh::fail(e == hipErrorOutOfMemory ? SH_ERR_OOM : SH_ERR_HIP,
                      "HIP error %d (%s) uploading an unpack plan", (int)e, hipGetErrorString(e));
    }
  }
  *out = plan;
  return SH_OK;
}

extern "C" int sh_plan_destroy(sh_plan* plan) {
  sh::clear_error();
  if (plan == nullptr) return SH_OK;
  int cur = -1;
  (void)hipGetDevice(&cur);
  if (plan->device >= 0 && cur != plan->device) (void)hipSetDevice(plan->device);
  hipError_t e1 = plan->d_descs ? hipFree(plan->d_descs) : hipSuccess;
  hipError_t e2 = plan->d_tile_map ? hipFree(plan->d_tile_map) : hipSuccess;
  if (plan->device >= 0 && cur >= 0 && cur != plan->device) (void)hipSetDevice(cur);
  delete plan;
  if (e1 != hipSuccess || e2 != hipSuccess)
    return sh::fail(SH_ERR_HIP, "HIP error %d freeing an unpack plan", (int)(e1 != hipSuccess ? e1 : e2));
  return SH_OK;
}

extern "C" int sh_plan_get_info(const sh_plan* plan, sh_plan_info* info) {
  sh::clear_error();
  if (plan == nullptr || info == nullptr) return sh::fail(SH_ERR_INVALID, "sh_plan_get_info: NULL argument");
  *info = plan->info;
  return SH_OK;
}

namespace {

// Checks the caller's buffers against a plan's extents (SH_OK or SH_ERR_INVALID).
int check_buffers(const sh_plan_info& in, const void* src, size_t src_bytes, const float* scales, size_t n_scale,
                  const void* dst, size_t dst_bytes, const char* who) {
  if (in.src_extent > 0 && (src == nullptr || src_bytes < in.src_extent))
    return sh::fail(SH_ERR_INVALID, "%s: source buffer of %zu bytes is smaller than the plan's %llu", who,
                    src == nullptr ? (size_t)0 : src_bytes, (unsigned long long)in.src_extent);
  if (dst == nullptr || dst_bytes < in.dst_extent)
    return sh::fail(SH_ERR_INVALID, "%s: destination buffer of %zu bytes is smaller than the plan's %llu", who,
                    dst == nullptr ? (size_t)0 : dst_bytes, (unsigned long long)in.dst_extent);
  const bool has_i8 = (in.kind_mask & (bit(SH_KIND_I8_ROWSCALE_BF16) | bit(SH_KIND_I8_ROWSCALE_F32))) != 0;
  if (has_i8 && (scales == nullptr || n_scale < in.scale_extent))
    return sh::fail(SH_ERR_INVALID, "%s: %zu scales given, the plan reads %llu", who,
                    scales == nullptr ? (size_t)0 : n_scale, (unsigned long long)in.scale_extent);
  return SH_OK;
}

// Launches the unpack kernel for a checked plan whose table and tile map are at d_descs /
// d_tile_map on the current device.
int launch_tiles(const sh_plan_info& in, const sh_unpack_desc* d_descs, const uint32_t* d_tile_map,
                 const void* src, const float* scales, const float* zps, void* dst, void* stream) {
  const bool has_i8 = (in.kind_mask & (bit(SH_KIND_I8_ROWSCALE_BF16) | bit(SH_KIND_I8_ROWSCALE_F32))) != 0;
  const bool has_zp = has_i8 && zps != nullptr;

  void (*kern)(SH_KERNEL_ARGS);
  if (in.kind_mask == kMaskDequantBf16)
    kern = has_zp ? sh_dequant_i8_bf16_zp_kernel : sh_dequant_i8_bf16_kernel;
  else if (in.kind_mask == kMaskCastBf16)
    kern = sh_cast_f32_bf16_kernel;
  else
    kern = has_zp ? sh_unpack_mixed_zp_kernel : sh_unpack_mixed_kernel;

  hipLaunchKernelGGL(kern, dim3(in.n_tiles), dim3(kThreads), 0, (hipStream_t)stream, d_descs, d_tile_map,
                     (const uint8_t*)src, scales, has_zp ? zps : nullptr, (uint8_t*)dst);
  SH_HIP(hipGetLastError());
  return SH_OK;
}

int launch(const sh_plan* plan, const void* src, size_t src_bytes, const float* scales,
           const float* zps, size_t n_scale, void* dst, size_t dst_bytes, void* stream,
           uint32_t required_mask, const char* who) {
  sh::clear_error();
  if (plan == nullptr) return sh::fail(SH_ERR_INVALID, "%s: plan is NULL", who);
  const sh_plan_info& in = plan->info;
  if (required_mask != 0 && (in.kind_mask & ~required_mask) != 0)
    return sh::fail(SH_ERR_INVALID, "%s: plan holds descriptor kinds (mask 0x%x) this entry point does not handle",
                    who, in.kind_mask);
  if (in.n_tiles == 0) return SH_OK;
  int cur = -1;
  SH_HIP(hipGetDevice(&cur));
  if (cur != plan->device)
    return sh::fail(SH_ERR_INVALID, "%s: plan was built on device %d but device %d is current", who,
                    plan->device, cur);
  if (int st = check_buffers(in, src, src_bytes, scales, n_scale, dst, dst_bytes, who)) return st;
  return launch_tiles(in, plan->d_descs, plan->d_tile_map, src, scales, zps, dst, stream);
}

// The scratch array's device address on the current device, looked up once per device.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_on_current_device(void** out, const char* who) {
  int dev = -1;
  SH_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return sh::fail(SH_ERR_INVALID, "%s: device %d out of range", who, dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return sh::fail(SH_ERR_HIP, "%s: hipGetSymbolAddress(scratch) on device %d: %s", who, dev,
                      hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SH_OK;
}

}  // namespace

extern "C" int sh_unpack(const sh_plan* plan, const void* src, size_t src_bytes, const float* scales,
                         const float* zero_points, size_t n_scale, void* dst, size_t dst_bytes,
                         void* stream) {
  return launch(plan, src, src_bytes, scales, zero_points, n_scale, dst, dst_bytes, stream, 0, "sh_unpack");
}

extern "C" int sh_dequant_i8_rowscale_bf16(const sh_plan* plan, const int8_t* src, size_t src_bytes,
                                           const float* scales, const float* zero_points, size_t n_scale,
                                           uint16_t* dst, size_t dst_bytes, void* stream) {
  return launch(plan, src, src_bytes, scales, zero_points, n_scale, dst, dst_bytes, stream, kMaskDequantBf16,
                "sh_dequant_i8_rowscale_bf16");
}

extern "C" int sh_unpack_cast_f32_bf16(const sh_plan* plan, const float* src, size_t src_bytes, uint16_t* dst,
                                       size_t dst_bytes, void* stream) {
  return launch(plan, src, src_bytes, nullptr, nullptr, 0, dst, dst_bytes, stream, kMaskCastBf16,
                "sh_unpack_cast_f32_bf16");
}

extern "C" int sh_unpack_noalloc(const sh_unpack_desc* descs, uint32_t n, const void* src, size_t src_bytes,
                                 const float* scales, const float* zero_points, size_t n_scale, void* dst,
                                 size_t dst_bytes, void* stream) {
  static const char* who = "sh_unpack_noalloc";
  sh::clear_error();
  thread_local std::vector<sh_unpack_desc> table;  // host side only, reused across calls
  sh_plan_info in{};
  if (int st = build_table(descs, n, table, in, who)) return st;
  if (table.size() > SH_UNPACK_NOALLOC_MAX_DESCS)
    return sh::fail(SH_ERR_INVALID, "%s: the plan needs %zu descriptors after splitting; at most %u fit the scratch",
                    who, table.size(), (unsigned)SH_UNPACK_NOALLOC_MAX_DESCS);
  if (in.n_tiles > SH_UNPACK_NOALLOC_MAX_TILES)
    return sh::fail(SH_ERR_INVALID, "%s: the plan needs %u tiles; at most %u fit the scratch", who, in.n_tiles,
                    (unsigned)SH_UNPACK_NOALLOC_MAX_TILES);
  if (in.n_tiles == 0) return SH_OK;
  if (int st = check_buffers(in, src, src_bytes, scales, n_scale, dst, dst_bytes, who)) return st;
  void* base = nullptr;
  if (int st = scratch_on_current_device(&base, who)) return st;
  sh_unpack_desc* d_descs = (sh_unpack_desc*)base;
  uint32_t* d_map = (uint32_t*)((uint8_t*)base + SH_UNPACK_NOALLOC_MAX_DESCS * sizeof(sh_unpack_desc));
  const hipStream_t s = (hipStream_t)stream;
  const uint32_t nd = (uint32_t)table.size();
  for (uint32_t first = 0; first < nd; first += kDescChunk) {
    DescChunk c{};
    c.first = first;
    c.count = std::min(kDescChunk, nd - first);
    std::copy(table.begin() + first, table.begin() + first + c.count, c.d);
    hipLaunchKernelGGL(sh_put_descs_kernel, dim3(1), dim3(kDescChunk), 0, s, c, d_descs);
  }
  hipLaunchKernelGGL(sh_fill_tile_map_kernel, dim3((in.n_tiles + 255) / 256), dim3(256), 0, s,
                     (const sh_unpack_desc*)d_descs, nd, d_map, in.n_tiles);
  SH_HIP(hipGetLastError());
  return launch_tiles(in, d_descs, d_map, src, scales, zero_points, dst, stream);
}

extern "C" int sh_index_div(uint32_t d, const uint32_t* n, uint32_t* q, size_t count) {
  sh::clear_error();
  if (d == 0) return sh::fail(SH_ERR_INVALID, "sh_index_div: divisor is 0");
  if (count > 0 && (n == nullptr || q == nullptr)) return sh::fail(SH_ERR_INVALID, "sh_index_div: NULL array");
  const uint64_t m = sh::udiv_magic(d);
  for (size_t i = 0; i < count; ++i) q[i] = sh::udiv(n[i], m);
  return SH_OK;
}
