// VMM residency allocator: slabs of reserved device address space whose
// regions are backed by physical memory on demand and unmapped under a VRAM
// ceiling.
//
// Behaviour follows the reference's Rust allocator (vmm_src/allocator.rs,
// eviction.rs, handle.rs, prefetch.rs, python.rs) on the HIP virtual memory
// API (hipMemAddressReserve / hipMemCreate / hipMemMap / hipMemSetAccess /
// hipMemUnmap / hipMemRelease):
//  * granularity = hipMemGetAllocationGranularity(RECOMMENDED); default
//    ceiling = total VRAM - max(2 GB, 15 %) (allocator.rs:101-115);
//  * a slab reserves its rounded size of address space; a region's size is
//    rounded up to the granularity and the slab's watermark starts at its
//    first region count (allocator.rs:140-198);
//  * ensure_resident: fast path on a Resident region is an atomic refcount
//    increment re-checked against the state (allocator.rs:213-276); the cold
//    path maps, evicting for space under the ceiling, and lowers the slab's
//    watermark (Watermarked) when nothing can be evicted (allocator.rs:282-468);
//  * eviction picks Resident, unreferenced regions by (slab priority, last
//    access) ascending, claims each by a state CAS and re-checks its refcount,
//    waits for the last consumer's event and lowers the watermark to the
//    evicted region (eviction.rs:15-144);
//  * set_priority re-opens the watermark of the highest-priority slab
//    (allocator.rs:505-533); a handle's release records an event on its stream
//    before dropping its reference (handle.rs:65-110);
//  * prefetch maps a region on a worker thread (prefetch.rs).
// Differences: every region reserves its own address range when it is defined
// (a slab is the group of its regions and bounds their offsets) — on gfx950
// with ROCm 7.2, hipMemSetAccess refuses (invalid argument) a mapping inside a
// reservation that already holds a mapping of another size, while separate
// reservations map any mix of sizes; the access clock and per-region last
// access are atomics (the reference's try_lock stamping can leave hot regions
// unstamped); a region must start at a granularity multiple and end inside its
// slab (checked when it is defined instead of failing at map time); mapping is
// synchronous on the host, so a prefetch needs no event; DLPack export uses
// kDLROCM.
#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <deque>
#include <memory>
#include <mutex>
#include <shared_mutex>
#include <thread>
#include <vector>

#include "sh_internal.h"

namespace {

enum : uint8_t { kUnmapped = SH_VMM_UNMAPPED, kResident = SH_VMM_RESIDENT };

struct VRegion {
  void* base = nullptr;  // the region's own address reservation
  uint64_t offset = 0, size = 0;
  std::atomic<uint8_t> state{kUnmapped};
  std::atomic<uint32_t> refcount{0};
  std::atomic<uint64_t> last_access{0};
  std::atomic<uint64_t> generation{0};  // bumped at every map: a new mapping holds no data
  std::mutex mu;  // phys and last_use
  hipMemGenericAllocationHandle_t phys{};
  bool has_phys = false;
  hipEvent_t last_use = nullptr;
  bool last_use_recorded = false;
};

struct VSlab {
  uint64_t size = 0;
  std::vector<std::unique_ptr<VRegion>> regions;
  std::atomic<uint32_t> priority{0};
  std::atomic<size_t> watermark{0};
};

}  // namespace

struct sh_vmm {
  sh::Live<sh::kLiveVmm> live;
  int device = 0;
  size_t granularity = 0;
  hipMemAllocationProp prop{};
  std::atomic<uint64_t> ceiling{0};
  std::atomic<uint64_t> clock{0};
  std::atomic<int> refs{1};  // the allocator itself + one per live handle
  std::shared_mutex slabs_mu;  // structure of `slabs` and of each slab's region list
  std::vector<std::unique_ptr<VSlab>> slabs;
  std::mutex cold_mu;  // mapping, eviction, mapped_bytes (taken before slabs_mu)
  uint64_t mapped_bytes = 0;
  uint64_t maps = 0, evictions = 0, unmap_failures = 0;
  int last_unmap_error = 0;
  // prefetch worker
  std::thread worker;
  std::mutex q_mu;
  std::condition_variable q_cv;
  std::deque<std::pair<uint32_t, uint32_t>> queue;
  bool stop = false;
};

struct sh_vmm_handle {
  sh_vmm* vmm = nullptr;
  uint32_t slab = 0, region = 0;
  uint64_t generation = 0;
  void* ptr = nullptr;
  hipStream_t stream = nullptr;
  bool released = false;
};

namespace {

uint64_t round_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

void unmap_region(VRegion& r) {
  std::lock_guard<std::mutex> g(r.mu);
  if (r.has_phys) {
    (void)hipMemUnmap(r.base, r.size);
    (void)hipMemRelease(r.phys);
    r.has_phys = false;
  }
}

void free_region(VRegion& r) {
  if (r.last_use) {
    (void)hipEventSynchronize(r.last_use);
    (void)hipEventDestroy(r.last_use);
    r.last_use = nullptr;
  }
  unmap_region(r);
  if (r.base) {
    (void)hipMemAddressFree(r.base, r.size);
    r.base = nullptr;
  }
}

void free_everything(sh_vmm* v) {
  (void)hipSetDevice(v->device);
  for (auto& sp : v->slabs) {
    if (!sp) continue;
    for (auto& rp : sp->regions) free_region(*rp);
  }
  v->slabs.clear();
}

void drop_ref(sh_vmm* v) {
  if (v->refs.fetch_sub(1, std::memory_order_acq_rel) == 1) {
    free_everything(v);
    delete v;
  }
}

// Caller holds cold_mu and a shared lock on slabs_mu.
int map_region(sh_vmm* v, VRegion& r) {
  hipMemGenericAllocationHandle_t h{};
  SH_HIP(hipMemCreate(&h, r.size, &v->prop, 0));
  void* p = r.base;
  hipError_t e = hipMemMap(p, r.size, 0, h, 0);
  if (e != hipSuccess) {
    (void)hipMemRelease(h);
    return sh::fail(SH_ERR_HIP, "HIP error %d (%s) in hipMemMap", (int)e, hipGetErrorString(e));
  }
  hipMemAccessDesc acc{};
  acc.location.type = hipMemLocationTypeDevice;
  acc.location.id = v->device;
  acc.flags = hipMemAccessFlagsProtReadWrite;
  e = hipMemSetAccess(p, r.size, &acc, 1);
  if (e != hipSuccess) {
    (void)hipMemUnmap(p, r.size);
    (void)hipMemRelease(h);
    return sh::fail(SH_ERR_HIP, "HIP error %d (%s) in hipMemSetAccess", (int)e, hipGetErrorString(e));
  }
  {
    std::lock_guard<std::mutex> g(r.mu);
    r.phys = h;
    r.has_phys = true;
  }
  r.last_access.store(v->clock.fetch_add(1) + 1, std::memory_order_relaxed);
  r.generation.fetch_add(1, std::memory_order_acq_rel);
  r.state.store(kResident, std::memory_order_release);
  v->mapped_bytes += r.size;
  v->maps++;
  return SH_OK;
}

// Frees at least `needed` bytes under the ceiling. Caller holds cold_mu and a
// shared lock on slabs_mu. SH_ERR_WATERMARK when not enough can be evicted.
int evict_for_space(sh_vmm* v, uint64_t needed) {
  const uint64_t ceiling = v->ceiling.load(std::memory_order_acquire);
  const uint64_t must = v->mapped_bytes + needed > ceiling ? v->mapped_bytes + needed - ceiling : 0;
  if (must == 0) return SH_OK;
  struct Cand { uint32_t prio; uint64_t access; size_t s, r; };
  std::vector<Cand> cands;
  for (size_t si = 0; si < v->slabs.size(); ++si) {
    VSlab* s = v->slabs[si].get();
    if (!s) continue;
    for (size_t ri = 0; ri < s->regions.size(); ++ri) {
      VRegion& r = *s->regions[ri];
      if (r.state.load(std::memory_order_acquire) == kResident && r.refcount.load(std::memory_order_acquire) == 0)
        cands.push_back({s->priority.load(), r.last_access.load(), si, ri});
    }
  }
  std::sort(cands.begin(), cands.end(), [](const Cand& a, const Cand& b) {
    return a.prio != b.prio ? a.prio < b.prio : a.access < b.access;
  });
  uint64_t freed = 0;
  for (const Cand& c : cands) {
    VSlab& s = *v->slabs[c.s];
    VRegion& r = *s.regions[c.r];
    if (r.refcount.load(std::memory_order_acquire) != 0) continue;
    uint8_t expect = kResident;
    // Claim, then re-check the refcount. A fast-path ensure_resident increments the refcount,
    // then re-checks the state: each side stores one atomic and then loads the other, so both
    // orders are seq_cst — with acquire/release alone both loads could miss the other's store
    // and the region be unmapped under a handle.
    if (!r.state.compare_exchange_strong(expect, kUnmapped, std::memory_order_seq_cst)) continue;
    if (r.refcount.load(std::memory_order_seq_cst) != 0) {
      r.state.store(kResident, std::memory_order_release);
      continue;
    }
    {
      std::lock_guard<std::mutex> g(r.mu);
      if (r.last_use && r.last_use_recorded) (void)hipEventSynchronize(r.last_use);
      r.last_use_recorded = false;
      if (r.has_phys) {
        hipError_t e = hipMemUnmap(r.base, r.size);
        if (e != hipSuccess) {
          v->unmap_failures++;
          v->last_unmap_error = (int)e;
          r.state.store(kResident, std::memory_order_release);
          continue;
        }
        (void)hipMemRelease(r.phys);
        r.has_phys = false;
      }
    }
    v->mapped_bytes -= r.size;
    v->evictions++;
    size_t wm = s.watermark.load(std::memory_order_acquire);
    if (c.r < wm) s.watermark.store(c.r, std::memory_order_release);
    freed += r.size;
    if (freed >= must) return SH_OK;
  }
  return sh::fail(SH_ERR_WATERMARK, "No evictable regions — all in use");
}

int lookup(sh_vmm* v, uint32_t slab, uint32_t region, VSlab** s, VRegion** r) {
  if (slab >= v->slabs.size() || !v->slabs[slab]) return sh::fail(SH_ERR_INVALID, "Invalid slab ID %u", slab);
  *s = v->slabs[slab].get();
  if (region >= (*s)->regions.size()) return sh::fail(SH_ERR_INVALID, "Invalid region ID %u", region);
  *r = (*s)->regions[region].get();
  return SH_OK;
}

sh_vmm_handle* make_handle(sh_vmm* v, uint32_t slab, uint32_t region, void* ptr, hipStream_t stream,
                           uint64_t generation) {
  v->refs.fetch_add(1, std::memory_order_acq_rel);
  auto* h = new sh_vmm_handle();
  h->vmm = v;
  h->slab = slab;
  h->region = region;
  h->generation = generation;
  h->ptr = ptr;
  h->stream = stream;
  return h;
}

// Maps a region for the prefetch worker; errors are dropped (a later
// ensure_resident reports them).
void prefetch_one(sh_vmm* v, uint32_t slab, uint32_t region) {
  std::lock_guard<std::mutex> cg(v->cold_mu);
  std::shared_lock<std::shared_mutex> sg(v->slabs_mu);
  VSlab* s;
  VRegion* r;
  if (lookup(v, slab, region, &s, &r) != SH_OK) { sh::clear_error(); return; }
  if (region >= s->watermark.load(std::memory_order_acquire)) return;
  if (r->state.load(std::memory_order_acquire) == kResident) return;
  if (evict_for_space(v, r->size) != SH_OK) { sh::clear_error(); return; }
  if (map_region(v, *r) != SH_OK) sh::clear_error();
}

void worker_loop(sh_vmm* v) {
  sh::name_thread("sh-vmm-prefetch");
  (void)hipSetDevice(v->device);
  for (;;) {
    std::pair<uint32_t, uint32_t> req;
    {
      std::unique_lock<std::mutex> g(v->q_mu);
      v->q_cv.wait(g, [&] { return v->stop || !v->queue.empty(); });
      if (v->stop) return;
      req = v->queue.front();
      v->queue.pop_front();
    }
    prefetch_one(v, req.first, req.second);
  }
}

}  // namespace

extern "C" int sh_vmm_create(int device, uint64_t ceiling_bytes, sh_vmm** out) {
  sh::clear_error();
  if (!out) return sh::fail(SH_ERR_INVALID, "sh_vmm_create: null output");
  SH_HIP(hipSetDevice(device));
  int supported = 0;
  SH_HIP(hipDeviceGetAttribute(&supported, hipDeviceAttributeVirtualMemoryManagementSupported, device));
  if (!supported) return sh::fail(SH_ERR_STATE, "device %d does not support virtual memory management", device);
  auto v = std::make_unique<sh_vmm>();
  v->device = device;
  v->prop.type = hipMemAllocationTypePinned;
  v->prop.location.type = hipMemLocationTypeDevice;
  v->prop.location.id = device;
  SH_HIP(hipMemGetAllocationGranularity(&v->granularity, &v->prop, hipMemAllocationGranularityRecommended));
  if (v->granularity == 0) return sh::fail(SH_ERR_HIP, "zero allocation granularity");
  size_t free_b = 0, total_b = 0;
  SH_HIP(hipMemGetInfo(&free_b, &total_b));
  const uint64_t reserve = std::max<uint64_t>(2ull << 30, (uint64_t)total_b * 15 / 100);
  v->ceiling.store(ceiling_bytes ? ceiling_bytes : (total_b > reserve ? total_b - reserve : 0));
  sh_vmm* raw = v.release();
  raw->worker = std::thread(worker_loop, raw);
  *out = raw;
  return SH_OK;
}

extern "C" int sh_vmm_destroy(sh_vmm* v) {
  sh::clear_error();
  if (!v) return SH_OK;
  {
    std::lock_guard<std::mutex> g(v->q_mu);
    v->stop = true;
  }
  v->q_cv.notify_all();
  if (v->worker.joinable()) v->worker.join();
  drop_ref(v);  // memory goes once the last handle is released too
  return SH_OK;
}

extern "C" int sh_vmm_info(sh_vmm* v, sh_vmm_stats* st) {
  sh::clear_error();
  if (!v || !st) return sh::fail(SH_ERR_INVALID, "sh_vmm_info: null argument");
  std::lock_guard<std::mutex> cg(v->cold_mu);
  std::shared_lock<std::shared_mutex> sg(v->slabs_mu);
  *st = sh_vmm_stats{};
  for (auto& s : v->slabs) {
    if (!s) continue;
    st->total_slabs++;
    st->total_regions += s->regions.size();
  }
  st->mapped_bytes = v->mapped_bytes;
  st->vram_ceiling = v->ceiling.load();
  st->granularity = v->granularity;
  st->maps = v->maps;
  st->evictions = v->evictions;
  st->unmap_failures = v->unmap_failures;
  st->last_unmap_error = (uint64_t)v->last_unmap_error;
  return SH_OK;
}

extern "C" int sh_vmm_create_slab(sh_vmm* v, uint64_t size, uint32_t* slab) {
  sh::clear_error();
  if (!v || !slab) return sh::fail(SH_ERR_INVALID, "sh_vmm_create_slab: null argument");
  if (size == 0) return sh::fail(SH_ERR_INVALID, "slab size must be positive");
  auto s = std::make_unique<VSlab>();
  s->size = round_up(size, v->granularity);
  std::unique_lock<std::shared_mutex> g(v->slabs_mu);
  for (size_t i = 0; i < v->slabs.size(); ++i) {
    if (!v->slabs[i]) {
      v->slabs[i] = std::move(s);
      *slab = (uint32_t)i;
      return SH_OK;
    }
  }
  v->slabs.push_back(std::move(s));
  *slab = (uint32_t)(v->slabs.size() - 1);
  return SH_OK;
}

extern "C" int sh_vmm_define_region(sh_vmm* v, uint32_t slab, uint64_t offset, uint64_t size, uint32_t* region) {
  sh::clear_error();
  if (!v || !region) return sh::fail(SH_ERR_INVALID, "sh_vmm_define_region: null argument");
  std::unique_lock<std::shared_mutex> g(v->slabs_mu);
  if (slab >= v->slabs.size() || !v->slabs[slab]) return sh::fail(SH_ERR_INVALID, "Invalid slab ID %u", slab);
  VSlab& s = *v->slabs[slab];
  const uint64_t rounded = round_up(size ? size : 1, v->granularity);
  if (offset % v->granularity)
    return sh::fail(SH_ERR_INVALID, "region offset %llu is not a multiple of the granularity %zu",
                    (unsigned long long)offset, v->granularity);
  if (offset + rounded > s.size)
    return sh::fail(SH_ERR_INVALID, "region [%llu, %llu) does not fit slab %u of %llu bytes",
                    (unsigned long long)offset, (unsigned long long)(offset + rounded), slab,
                    (unsigned long long)s.size);
  auto r = std::make_unique<VRegion>();
  r->offset = offset;
  r->size = rounded;
  SH_HIP(hipSetDevice(v->device));
  SH_HIP(hipMemAddressReserve(&r->base, rounded, v->granularity, nullptr, 0));
  hipError_t e = hipEventCreateWithFlags(&r->last_use, hipEventDisableTiming);
  if (e != hipSuccess) {
    (void)hipMemAddressFree(r->base, rounded);
    return sh::fail(SH_ERR_HIP, "HIP error %d (%s) in hipEventCreateWithFlags", (int)e, hipGetErrorString(e));
  }
  s.regions.push_back(std::move(r));
  if (s.watermark.load() == 0) s.watermark.store(s.regions.size());
  *region = (uint32_t)(s.regions.size() - 1);
  return SH_OK;
}

extern "C" int sh_vmm_ensure_resident(sh_vmm* v, uint32_t slab, uint32_t region, void* stream, sh_vmm_handle** out) {
  sh::clear_error();
  if (!v || !out) return sh::fail(SH_ERR_INVALID, "sh_vmm_ensure_resident: null argument");
  hipStream_t st = static_cast<hipStream_t>(stream);
  {  // fast path: shared lock and atomics only
    std::shared_lock<std::shared_mutex> sg(v->slabs_mu);
    VSlab* s;
    VRegion* r;
    int rc = lookup(v, slab, region, &s, &r);
    if (rc != SH_OK) return rc;
    if (region >= s->watermark.load(std::memory_order_acquire))
      return sh::fail(SH_ERR_WATERMARK, "Region watermarked — use fallback path");
    if (r->state.load(std::memory_order_acquire) == kResident) {
      // seq_cst store-then-load, paired with the evictor's claim-then-recheck (evict_for_space)
      r->refcount.fetch_add(1, std::memory_order_seq_cst);
      if (r->state.load(std::memory_order_seq_cst) == kResident) {
        r->last_access.store(v->clock.fetch_add(1) + 1, std::memory_order_relaxed);
        *out = make_handle(v, slab, region, r->base, st, r->generation.load());
        return SH_OK;
      }
      r->refcount.fetch_sub(1, std::memory_order_acq_rel);  // lost to an eviction
    }
  }
  // cold path
  std::lock_guard<std::mutex> cg(v->cold_mu);
  std::shared_lock<std::shared_mutex> sg(v->slabs_mu);
  VSlab* s;
  VRegion* r;
  int rc = lookup(v, slab, region, &s, &r);
  if (rc != SH_OK) return rc;
  if (region >= s->watermark.load(std::memory_order_acquire))
    return sh::fail(SH_ERR_WATERMARK, "Region watermarked — use fallback path");
  SH_HIP(hipSetDevice(v->device));
  if (r->state.load(std::memory_order_acquire) != kResident) {
    rc = evict_for_space(v, r->size);
    if (rc != SH_OK) {
      size_t wm = s->watermark.load(std::memory_order_acquire);
      if (region < wm) s->watermark.store(region, std::memory_order_release);
      return sh::fail(SH_ERR_WATERMARK, "Region watermarked — use fallback path");
    }
    rc = map_region(v, *r);
    if (rc != SH_OK) return rc;
  }
  r->refcount.fetch_add(1, std::memory_order_acq_rel);
  r->last_access.store(v->clock.fetch_add(1) + 1, std::memory_order_relaxed);
  *out = make_handle(v, slab, region, r->base, st, r->generation.load());
  return SH_OK;
}

extern "C" int sh_vmm_time_fast_path(sh_vmm* v, uint32_t slab, uint32_t region, void* stream, uint32_t iters,
                                     double* out2) {
  sh::clear_error();
  if (!v || !out2 || iters == 0) return sh::fail(SH_ERR_INVALID, "sh_vmm_time_fast_path: bad argument");
  using clk = std::chrono::steady_clock;
  sh_vmm_handle* h = nullptr;
  // the region resident (the cold path maps it if needed) and the code paths warm
  if (int st = sh_vmm_ensure_resident(v, slab, region, stream, &h)) return st;
  sh_vmm_handle_destroy(h);
  std::vector<sh_vmm_handle*> held;
  held.reserve(iters);
  auto t0 = clk::now();
  for (uint32_t i = 0; i < iters; ++i) {
    if (int st = sh_vmm_ensure_resident(v, slab, region, stream, &h)) {
      for (sh_vmm_handle* x : held) sh_vmm_handle_destroy(x);
      return st;
    }
    held.push_back(h);
  }
  auto t1 = clk::now();
  for (sh_vmm_handle* x : held) sh_vmm_handle_destroy(x);
  auto t2 = clk::now();
  for (uint32_t i = 0; i < iters; ++i) {
    if (int st = sh_vmm_ensure_resident(v, slab, region, stream, &h)) return st;
    sh_vmm_handle_destroy(h);
  }
  auto t3 = clk::now();
  out2[0] = std::chrono::duration<double, std::nano>(t1 - t0).count() / iters;
  out2[1] = std::chrono::duration<double, std::nano>(t3 - t2).count() / iters;
  return SH_OK;
}

extern "C" int sh_vmm_prefetch(sh_vmm* v, uint32_t slab, uint32_t region) {
  sh::clear_error();
  if (!v) return sh::fail(SH_ERR_INVALID, "sh_vmm_prefetch: null allocator");
  {
    std::shared_lock<std::shared_mutex> sg(v->slabs_mu);
    VSlab* s;
    VRegion* r;
    if (lookup(v, slab, region, &s, &r) != SH_OK) { sh::clear_error(); return SH_OK; }
    if (region >= s->watermark.load() || r->state.load() == kResident) return SH_OK;
  }
  {
    std::lock_guard<std::mutex> g(v->q_mu);
    v->queue.emplace_back(slab, region);
  }
  v->q_cv.notify_one();
  return SH_OK;
}

extern "C" int sh_vmm_set_priority(sh_vmm* v, uint32_t slab, uint32_t priority) {
  sh::clear_error();
  if (!v) return sh::fail(SH_ERR_INVALID, "sh_vmm_set_priority: null allocator");
  std::unique_lock<std::shared_mutex> g(v->slabs_mu);
  if (slab >= v->slabs.size() || !v->slabs[slab]) return sh::fail(SH_ERR_INVALID, "Invalid slab ID %u", slab);
  v->slabs[slab]->priority.store(priority);
  VSlab* top = nullptr;
  for (auto& s : v->slabs)
    if (s && (!top || s->priority.load() > top->priority.load())) top = s.get();
  if (top) top->watermark.store(top->regions.size());
  return SH_OK;
}

extern "C" int sh_vmm_set_ceiling(sh_vmm* v, uint64_t ceiling_bytes) {
  sh::clear_error();
  if (!v) return sh::fail(SH_ERR_INVALID, "sh_vmm_set_ceiling: null allocator");
  v->ceiling.store(ceiling_bytes, std::memory_order_release);
  return SH_OK;
}

extern "C" int sh_vmm_destroy_slab(sh_vmm* v, uint32_t slab) {
  sh::clear_error();
  if (!v) return sh::fail(SH_ERR_INVALID, "sh_vmm_destroy_slab: null allocator");
  std::lock_guard<std::mutex> cg(v->cold_mu);
  std::unique_lock<std::shared_mutex> g(v->slabs_mu);
  if (slab >= v->slabs.size() || !v->slabs[slab]) return sh::fail(SH_ERR_INVALID, "Invalid slab ID %u", slab);
  VSlab& s = *v->slabs[slab];
  for (auto& r : s.regions)
    if (r->refcount.load() > 0) return sh::fail(SH_ERR_STATE, "Slab has active handles");
  SH_HIP(hipSetDevice(v->device));
  for (auto& r : s.regions) {
    if (r->state.load() == kResident) v->mapped_bytes -= r->size;
    free_region(*r);
    r->state.store(kUnmapped);
  }
  v->slabs[slab].reset();
  return SH_OK;
}

extern "C" int sh_vmm_region_info(sh_vmm* v, uint32_t slab, uint32_t region, sh_vmm_region_stats* st) {
  sh::clear_error();
  if (!v || !st) return sh::fail(SH_ERR_INVALID, "sh_vmm_region_info: null argument");
  std::shared_lock<std::shared_mutex> sg(v->slabs_mu);
  VSlab* s;
  VRegion* r;
  int rc = lookup(v, slab, region, &s, &r);
  if (rc != SH_OK) return rc;
  st->state = r->state.load();
  st->refcount = r->refcount.load();
  st->offset = r->offset;
  st->size = r->size;
  st->last_access = r->last_access.load();
  st->watermark = s->watermark.load();
  st->priority = s->priority.load();
  return SH_OK;
}

extern "C" int sh_vmm_handle_ptr(sh_vmm_handle* h, void** ptr) {
  sh::clear_error();
  if (!h || !ptr) return sh::fail(SH_ERR_INVALID, "sh_vmm_handle_ptr: null argument");
  if (h->released) return sh::fail(SH_ERR_STATE, "Handle already released");
  *ptr = h->ptr;
  return SH_OK;
}

extern "C" int sh_vmm_handle_generation(sh_vmm_handle* h, uint64_t* generation) {
  sh::clear_error();
  if (!h || !generation) return sh::fail(SH_ERR_INVALID, "sh_vmm_handle_generation: null argument");
  *generation = h->generation;
  return SH_OK;
}

extern "C" int sh_vmm_handle_release(sh_vmm_handle* h) {
  sh::clear_error();
  if (!h) return sh::fail(SH_ERR_INVALID, "sh_vmm_handle_release: null handle");
  if (h->released) return sh::fail(SH_ERR_STATE, "Handle already released");
  sh_vmm* v = h->vmm;
  {
    std::shared_lock<std::shared_mutex> sg(v->slabs_mu);
    VSlab* s;
    VRegion* r;
    if (lookup(v, h->slab, h->region, &s, &r) == SH_OK) {
      std::lock_guard<std::mutex> g(r->mu);
      // the region may be unmapped only after the work queued on the consumer's stream
      if (r->last_use && hipEventRecord(r->last_use, h->stream) == hipSuccess) r->last_use_recorded = true;
      r->refcount.fetch_sub(1, std::memory_order_acq_rel);
    } else {
      sh::clear_error();
    }
  }
  h->released = true;
  drop_ref(v);
  return SH_OK;
}

extern "C" int sh_vmm_handle_destroy(sh_vmm_handle* h) {
  sh::clear_error();
  if (!h) return SH_OK;
  if (!h->released) sh_vmm_handle_release(h);
  delete h;
  return SH_OK;
}

// ── DLPack export ─────────────────────────────────────────────────────────

namespace {

struct DLPackCtx {
  sh_vmm_handle* handle;
  std::vector<int64_t> shape;
};

void dl_deleter(sh_dl_managed_tensor* t) {
  if (!t) return;
  auto* ctx = static_cast<DLPackCtx*>(t->manager_ctx);
  if (ctx) {
    sh_vmm_handle_destroy(ctx->handle);
    delete ctx;
  }
  delete t;
}

}  // namespace

extern "C" int sh_vmm_handle_export(sh_vmm_handle* h, uint8_t code, uint8_t bits, int32_t ndim, const int64_t* shape,
                                    sh_dl_managed_tensor** out) {
  sh::clear_error();
  if (!h || !out || ndim < 0 || (ndim && !shape)) return sh::fail(SH_ERR_INVALID, "sh_vmm_handle_export: bad argument");
  if (h->released) return sh::fail(SH_ERR_STATE, "Handle already released");
  if (bits == 0 || bits % 8) return sh::fail(SH_ERR_INVALID, "dtype bits must be a positive multiple of 8");
  uint64_t numel = 1;
  for (int32_t i = 0; i < ndim; ++i) {
    if (shape[i] < 0) return sh::fail(SH_ERR_INVALID, "negative dimension");
    numel *= (uint64_t)shape[i];
  }
  sh_vmm* v = h->vmm;
  sh_vmm_handle* dup = nullptr;
  {
    std::shared_lock<std::shared_mutex> sg(v->slabs_mu);
    VSlab* s;
    VRegion* r;
    int rc = lookup(v, h->slab, h->region, &s, &r);
    if (rc != SH_OK) return rc;
    if (numel * (bits / 8) > r->size)
      return sh::fail(SH_ERR_INVALID, "%llu bytes do not fit region of %llu bytes",
                      (unsigned long long)(numel * (bits / 8)), (unsigned long long)r->size);
    if (r->state.load() != kResident) return sh::fail(SH_ERR_INVALID, "region is not resident");
    // the tensor holds a reference of its own (python.rs:137-183)
    r->refcount.fetch_add(1, std::memory_order_acq_rel);
    dup = make_handle(v, h->slab, h->region, h->ptr, h->stream, h->generation);
  }
  auto* ctx = new DLPackCtx{dup, std::vector<int64_t>(shape, shape + ndim)};
  auto* t = new sh_dl_managed_tensor();
  t->dl_tensor.data = h->ptr;
  t->dl_tensor.device.device_type = SH_DL_ROCM;
  t->dl_tensor.device.device_id = v->device;
  t->dl_tensor.ndim = ndim;
  t->dl_tensor.dtype.code = code;
  t->dl_tensor.dtype.bits = bits;
  t->dl_tensor.dtype.lanes = 1;
  t->dl_tensor.shape = ctx->shape.data();
  t->dl_tensor.strides = nullptr;
  t->dl_tensor.byte_offset = 0;
  t->manager_ctx = ctx;
  t->deleter = dl_deleter;
  *out = t;
  return SH_OK;
}

extern "C" int sh_dl_free(sh_dl_managed_tensor* t) {
  sh::clear_error();
  if (t && t->deleter) t->deleter(t);
  return SH_OK;
}
