// Unpack plans and launches (host side): validates a block's descriptors, cuts oversize regions,
// assigns tiles, uploads the launch table and tile map, and launches the kernels of
// sh_unpack.hip (loaded from the library's code object, sh_kernels.cpp).
//
// Replaces the host-side staging arithmetic of the reference:
//   SquareQ dequant   src/stagehand/scheduler.py:290-300
//   bias / param cast src/stagehand/scheduler.py:181, 224-230, 302-306, 1066-1071
//   zero-fill         src/stagehand/scheduler.py:240, 276-297, 325

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <new>
#include <vector>

#include "sh_internal.h"
#include "sh_unpack_shape.h"
#include "stagehand_native.h"

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
                 const void* src, const float* scales, const float* zps, void* dst, void* stream, const char* who) {
  const bool has_i8 = (in.kind_mask & (bit(SH_KIND_I8_ROWSCALE_BF16) | bit(SH_KIND_I8_ROWSCALE_F32))) != 0;
  const bool has_zp = has_i8 && zps != nullptr;

  sh::KernelId kern;
  if (in.kind_mask == kMaskDequantBf16)
    kern = has_zp ? sh::kKernDequantBf16Zp : sh::kKernDequantBf16;
  else if (in.kind_mask == kMaskCastBf16)
    kern = sh::kKernCastBf16;
  else
    kern = has_zp ? sh::kKernMixedZp : sh::kKernMixed;

  const uint8_t* src_b = (const uint8_t*)src;
  const float* zp_arg = has_zp ? zps : nullptr;
  uint8_t* dst_b = (uint8_t*)dst;
  void* args[] = {(void*)&d_descs, (void*)&d_tile_map, (void*)&src_b, (void*)&scales, (void*)&zp_arg, (void*)&dst_b};
  return sh::launch_kernel(kern, in.n_tiles, kThreads, (hipStream_t)stream, args, who);
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
  return launch_tiles(in, plan->d_descs, plan->d_tile_map, src, scales, zps, dst, stream, who);
}

// sh_unpack_noalloc's state. One lock orders the host side of every call; per device, an
// event recorded after the last call's launches. Every call first makes its stream wait for
// that event, so its writes to the device's scratch array start only after the previous call's
// kernels have read it, whichever streams or threads the calls come from (on one stream the
// wait costs nothing on the device). Nothing here has a destructor: the table is never freed (it
// holds at most the largest plan seen) and the events end in sh_shutdown.
constexpr int kMaxDevices = 64;
struct NoallocDevice {
  hipEvent_t done = nullptr;
  bool pending = false;  // `done` has been recorded after a call's launches
};
std::mutex g_noalloc_mu;
std::vector<sh_unpack_desc>* g_noalloc_table = nullptr;
NoallocDevice g_noalloc_dev[kMaxDevices];

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
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  if (g_noalloc_table == nullptr) {
    g_noalloc_table = new (std::nothrow) std::vector<sh_unpack_desc>();
    if (g_noalloc_table == nullptr) return sh::fail(SH_ERR_OOM, "%s: out of host memory", who);
  }
  std::vector<sh_unpack_desc>& table = *g_noalloc_table;
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
  int dev = -1;
  SH_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return sh::fail(SH_ERR_INVALID, "%s: device %d out of range", who, dev);
  void* base = nullptr;
  if (int st = sh::noalloc_scratch(&base, who)) return st;
  NoallocDevice& nd_state = g_noalloc_dev[dev];
  if (nd_state.done == nullptr) SH_HIP(hipEventCreateWithFlags(&nd_state.done, hipEventDisableTiming));
  const hipStream_t s = (hipStream_t)stream;
  // Under stream capture the launches run only when the graph is replayed; ordering a replay
  // with other calls on this GPU is the caller's (the event is neither waited on nor recorded).
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  SH_HIP(hipStreamIsCapturing(s, &capture));
  const bool eager = capture == hipStreamCaptureStatusNone;
  if (eager && nd_state.pending) SH_HIP(hipStreamWaitEvent(s, nd_state.done, 0));

  sh_unpack_desc* d_descs = (sh_unpack_desc*)base;
  uint32_t* d_map = (uint32_t*)((uint8_t*)base + SH_UNPACK_NOALLOC_MAX_DESCS * sizeof(sh_unpack_desc));
  const uint32_t nd = (uint32_t)table.size();
  int st = SH_OK;
  bool queued = false;
  for (uint32_t first = 0; first < nd && st == SH_OK; first += kDescChunk) {
    DescChunk c{};
    c.first = first;
    c.count = std::min(kDescChunk, nd - first);
    std::copy(table.begin() + first, table.begin() + first + c.count, c.d);
    void* args[] = {(void*)&c, (void*)&d_descs};
    st = sh::launch_kernel(sh::kKernPutDescs, 1, kDescChunk, s, args, who);
    queued |= st == SH_OK;
  }
  if (st == SH_OK) {
    const sh_unpack_desc* table_arg = d_descs;
    uint32_t tiles = in.n_tiles;
    void* args[] = {(void*)&table_arg, (void*)&nd, (void*)&d_map, (void*)&tiles};
    st = sh::launch_kernel(sh::kKernFillTileMap, (in.n_tiles + 255) / 256, 256, s, args, who);
  }
  if (st == SH_OK) st = launch_tiles(in, d_descs, d_map, src, scales, zero_points, dst, stream, who);
  if (eager && queued) {
    // Recorded after whatever was queued, also when a later launch failed: the next call must
    // not overwrite a table that a queued kernel may still read.
    const hipError_t e = hipEventRecord(nd_state.done, s);
    if (e == hipSuccess) {
      nd_state.pending = true;
    } else if (st == SH_OK) {
      st = sh::fail(SH_ERR_HIP, "%s: hipEventRecord: HIP error %d (%s)", who, (int)e, hipGetErrorString(e));
    }
  }
  return st;
}

void sh::noalloc_release() {
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  for (NoallocDevice& d : g_noalloc_dev) {
    if (d.done != nullptr) (void)hipEventDestroy(d.done);
    d = NoallocDevice{};
  }
}

extern "C" int sh_index_div(uint32_t d, const uint32_t* n, uint32_t* q, size_t count) {
  sh::clear_error();
  if (d == 0) return sh::fail(SH_ERR_INVALID, "sh_index_div: divisor is 0");
  if (count > 0 && (n == nullptr || q == nullptr)) return sh::fail(SH_ERR_INVALID, "sh_index_div: NULL array");
  const uint64_t m = sh::udiv_magic(d);
  for (size_t i = 0; i < count; ++i) q[i] = sh::udiv(n[i], m);
  return SH_OK;
}
