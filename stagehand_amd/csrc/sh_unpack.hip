// Slab unpack kernels for gfx950: SquareQ INT8→bf16 dequant and fp32→bf16
// cast, scattering a packed device-resident source slab into a block's
// contiguous parameter buffer. Device code only: built into a code object that
// the library embeds and loads with the module API (sh_kernels.cpp); the plans
// and launches are host code in sh_unpack.cpp.
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

#include <cstdint>
#include <cstring>

#include "sh_internal.h"
#include "sh_unpack_shape.h"
#include "stagehand_native.h"

#pragma clang fp contract(off)

namespace {

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
// GPU (each device's load of the code object holds its own), until the library unloads its
// kernels: descriptors at offset 0, the tile map after them. The host never names this
// array: it looks up the device address by name in the loaded module (hipModuleGetGlobal,
// sh_kernels.cpp), so the symbol has external C linkage.
static_assert(SH_UNPACK_NOALLOC_SCRATCH_BYTES ==
                  SH_UNPACK_NOALLOC_MAX_DESCS * sizeof(sh_unpack_desc) + SH_UNPACK_NOALLOC_MAX_TILES * 4ull,
              "scratch layout: descriptor table, then one uint32 per tile");
extern "C" {
__device__ __align__(256) uint8_t scratch[SH_UNPACK_NOALLOC_SCRATCH_BYTES];
}

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
