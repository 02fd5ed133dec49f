// Fixed pinned host slab pool with event-fenced release, and a small thread
// pool for multi-threaded host copies into slabs.
//
// Pool semantics follow src/stagehand/pool.py:42-246: N equal slabs allocated
// once (never grows), acquire blocks while none is free, stats count
// total/free/in_use/peak_in_use/wait_count/total_wait_ms. Two additions serve
// the device path: (1) a slab may be released *after* the work queued so far
// on a stream (sh_pool_release_after): the pool records its own event and
// hands the slab out again only once that event has completed, so the host
// never waits for an H2D copy just to recycle its source slab; (2) the pool
// allocates one hipHostMalloc region (pinned, coherent) or, when asked for
// unpinned memory (no GPU), one aligned malloc region.
//
// All entry points are thread safe. Blocking calls are made through ctypes,
// which releases the Python GIL for their duration.

#include <hip/hip_runtime.h>
#include <pthread.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <functional>
#include <memory>
#include <mutex>
#include <new>
#include <thread>
#include <vector>

#include "sh_internal.h"
#include "stagehand_native.h"

struct sh_pool {
  sh::Live<sh::kLivePool> live;
  uint8_t* base = nullptr;
  uint64_t slab_bytes = 0;
  uint32_t num_slabs = 0;
  int pinned = 0;
  std::mutex mu;
  std::condition_variable cv;
  std::deque<uint32_t> free_list;
  struct Fenced {
    uint32_t slab;
    hipEvent_t ev;
  };
  std::deque<Fenced> fenced;        // released after an event, in release order
  std::vector<hipEvent_t> spare_events;
  std::vector<uint8_t> held;        // 1 while acquired or fenced
  uint64_t in_use = 0, peak_in_use = 0, wait_count = 0;
  double total_wait_ms = 0.0;
  bool shutdown = false;
};

namespace {

// Moves fenced slabs whose events have completed to the free list. Caller holds mu.
void reclaim_locked(sh_pool* p) {
  while (!p->fenced.empty()) {
    sh_pool::Fenced f = p->fenced.front();
    const hipError_t e = hipEventQuery(f.ev);
    if (e == hipErrorNotReady) break;
    p->fenced.pop_front();
    p->spare_events.push_back(f.ev);
    p->free_list.push_back(f.slab);
    p->held[f.slab] = 0;
    p->in_use -= 1;
  }
}

}  // namespace

extern "C" int sh_pool_create(uint32_t num_slabs, uint64_t slab_bytes, int pinned, sh_pool** out) {
  sh::clear_error();
  if (out == nullptr) return sh::fail(SH_ERR_INVALID, "sh_pool_create: out is NULL");
  *out = nullptr;
  if (num_slabs == 0 || slab_bytes == 0) return sh::fail(SH_ERR_INVALID, "sh_pool_create: empty pool");
  if (slab_bytes > UINT64_MAX / num_slabs) return sh::fail(SH_ERR_INVALID, "sh_pool_create: size overflow");
  const uint64_t total = slab_bytes * num_slabs;
  sh_pool* p = new (std::nothrow) sh_pool();
  if (p == nullptr) return sh::fail(SH_ERR_OOM, "sh_pool_create: out of host memory");
  p->slab_bytes = slab_bytes;
  p->num_slabs = num_slabs;
  p->pinned = pinned ? 1 : 0;
  if (pinned) {
    void* mem = nullptr;
    const hipError_t e = hipHostMalloc(&mem, total, hipHostMallocDefault);
    if (e != hipSuccess) {
      delete p;
      return sh::fail(SH_ERR_OOM, "sh_pool_create: could not pin %llu bytes (HIP error %d: %s)",
                      (unsigned long long)total, (int)e, hipGetErrorString(e));
    }
    p->base = (uint8_t*)mem;
  } else {
    void* mem = nullptr;
    if (posix_memalign(&mem, 4096, total) != 0) {
      delete p;
      return sh::fail(SH_ERR_OOM, "sh_pool_create: could not allocate %llu bytes", (unsigned long long)total);
    }
    p->base = (uint8_t*)mem;
  }
  p->held.assign(num_slabs, 0);
  for (uint32_t i = 0; i < num_slabs; ++i) p->free_list.push_back(i);
  *out = p;
  return SH_OK;
}

extern "C" int sh_pool_destroy(sh_pool* p) {
  sh::clear_error();
  if (p == nullptr) return SH_OK;
  {
    std::lock_guard<std::mutex> lk(p->mu);
    p->shutdown = true;
    for (auto& f : p->fenced) {
      (void)hipEventSynchronize(f.ev);
      (void)hipEventDestroy(f.ev);
    }
    p->fenced.clear();
    for (hipEvent_t ev : p->spare_events) (void)hipEventDestroy(ev);
    p->spare_events.clear();
  }
  p->cv.notify_all();
  int status = SH_OK;
  if (p->pinned) {
    const hipError_t e = hipHostFree(p->base);
    if (e != hipSuccess) status = sh::fail(SH_ERR_HIP, "sh_pool_destroy: hipHostFree failed (%d)", (int)e);
  } else {
    free(p->base);
  }
  delete p;
  return status;
}

extern "C" int sh_pool_slab_ptr(sh_pool* p, uint32_t slab, void** ptr) {
  sh::clear_error();
  if (p == nullptr || ptr == nullptr) return sh::fail(SH_ERR_INVALID, "sh_pool_slab_ptr: NULL argument");
  if (slab >= p->num_slabs) return sh::fail(SH_ERR_INVALID, "sh_pool_slab_ptr: slab %u out of range", slab);
  *ptr = p->base + (uint64_t)slab * p->slab_bytes;
  return SH_OK;
}

extern "C" int sh_pool_acquire(sh_pool* p, int64_t timeout_ms, uint32_t* slab, double* waited_ms) {
  sh::clear_error();
  if (p == nullptr || slab == nullptr) return sh::fail(SH_ERR_INVALID, "sh_pool_acquire: NULL argument");
  const auto t0 = std::chrono::steady_clock::now();
  bool waited = false;
  std::unique_lock<std::mutex> lk(p->mu);
  for (;;) {
    if (p->shutdown) return sh::fail(SH_ERR_STATE, "sh_pool_acquire: pool is shut down");
    reclaim_locked(p);
    if (!p->free_list.empty()) break;
    waited = true;
    if (!p->fenced.empty()) {
      // The oldest fenced slab frees up when its copy completes: wait for it
      // without holding the lock.
      hipEvent_t ev = p->fenced.front().ev;
      lk.unlock();
      const hipError_t e = hipEventSynchronize(ev);
      lk.lock();
      if (e != hipSuccess) return sh::fail(SH_ERR_HIP, "sh_pool_acquire: hipEventSynchronize failed (%d)", (int)e);
      continue;
    }
    if (timeout_ms >= 0) {
      const auto deadline = t0 + std::chrono::milliseconds(timeout_ms);
      if (p->cv.wait_until(lk, deadline) == std::cv_status::timeout) {
        reclaim_locked(p);
        if (!p->free_list.empty()) break;
        return sh::fail(SH_ERR_TIMEOUT, "sh_pool_acquire: no slab became free within %lld ms", (long long)timeout_ms);
      }
    } else {
      p->cv.wait_for(lk, std::chrono::milliseconds(100));
    }
  }
  const uint32_t s = p->free_list.front();
  p->free_list.pop_front();
  p->held[s] = 1;
  p->in_use += 1;
  p->peak_in_use = std::max(p->peak_in_use, p->in_use);
  const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  if (waited) {
    p->wait_count += 1;
    p->total_wait_ms += ms;
  }
  if (waited_ms) *waited_ms = waited ? ms : 0.0;
  *slab = s;
  return SH_OK;
}

extern "C" int sh_pool_release(sh_pool* p, uint32_t slab) {
  sh::clear_error();
  if (p == nullptr) return sh::fail(SH_ERR_INVALID, "sh_pool_release: pool is NULL");
  {
    std::lock_guard<std::mutex> lk(p->mu);
    if (slab >= p->num_slabs || !p->held[slab])
      return sh::fail(SH_ERR_INVALID, "sh_pool_release: slab %u is not acquired from this pool", slab);
    p->held[slab] = 0;
    p->free_list.push_back(slab);
    p->in_use -= 1;
  }
  p->cv.notify_all();
  return SH_OK;
}

extern "C" int sh_pool_release_after(sh_pool* p, uint32_t slab, void* stream) {
  sh::clear_error();
  if (p == nullptr) return sh::fail(SH_ERR_INVALID, "sh_pool_release_after: pool is NULL");
  std::lock_guard<std::mutex> lk(p->mu);
  if (slab >= p->num_slabs || !p->held[slab])
    return sh::fail(SH_ERR_INVALID, "sh_pool_release_after: slab %u is not acquired from this pool", slab);
  hipEvent_t ev = nullptr;
  if (!p->spare_events.empty()) {
    ev = p->spare_events.back();
    p->spare_events.pop_back();
  } else {
    SH_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
  }
  const hipError_t e = hipEventRecord(ev, (hipStream_t)stream);
  if (e != hipSuccess) {
    p->spare_events.push_back(ev);
    return sh::fail(SH_ERR_HIP, "sh_pool_release_after: hipEventRecord failed (%d: %s)", (int)e, hipGetErrorString(e));
  }
  p->fenced.push_back({slab, ev});
  // held stays 1 until the event completes; reclaim_locked clears it.
  return SH_OK;
}

extern "C" int sh_pool_get_stats(sh_pool* p, sh_pool_stats* st) {
  sh::clear_error();
  if (p == nullptr || st == nullptr) return sh::fail(SH_ERR_INVALID, "sh_pool_get_stats: NULL argument");
  std::lock_guard<std::mutex> lk(p->mu);
  reclaim_locked(p);
  st->total = p->num_slabs;
  st->free = p->free_list.size();
  st->in_use = p->in_use;
  st->peak_in_use = p->peak_in_use;
  st->wait_count = p->wait_count;
  st->fenced = p->fenced.size();
  st->total_wait_ms = p->total_wait_ms;
  st->slab_bytes = p->slab_bytes;
  st->pinned = (uint64_t)p->pinned;
  return SH_OK;
}

// ── multi-threaded host copies ────────────────────────────────────────────

namespace {

class CopyPool {
 public:
  // The process-wide pool, created on first use. Without sh_shutdown it is never
  // destroyed: a static destructor joining the threads at process exit would race
  // with the HIP runtime's and other libraries' own teardown. sh_shutdown drops the
  // global reference instead; the pool's threads are joined when the last user
  // (sh_shutdown itself, or a parallel_for still running) lets go of it.
  static std::shared_ptr<CopyPool> acquire() {
    std::lock_guard<std::mutex> lk(global_mu());
    std::shared_ptr<CopyPool>& inst = global();
    if (!inst) inst.reset(new CopyPool());
    return inst;
  }
  static std::shared_ptr<CopyPool> take_global() {
    std::lock_guard<std::mutex> lk(global_mu());
    std::shared_ptr<CopyPool> out;
    out.swap(global());
    return out;
  }
  static int64_t running_threads() { return running_.load(); }

  ~CopyPool() {
    {
      std::lock_guard<std::mutex> lk(mu_);
      stop_ = true;
    }
    cv_.notify_all();
    for (std::thread& t : workers_)
      if (t.joinable()) t.join();
  }

  // Runs fn(i) for i in [0, n) on up to `threads` workers (caller included).
  void parallel_for(size_t n, unsigned threads, const std::function<void(size_t)>& fn) {
    threads = std::max(1u, std::min<unsigned>(threads, (unsigned)workers_.size() + 1));
    if (n == 0) return;
    if (threads == 1 || n == 1) {
      for (size_t i = 0; i < n; ++i) fn(i);
      return;
    }
    std::lock_guard<std::mutex> serial(run_mu_);
    std::atomic<size_t> next{0};
    std::atomic<unsigned> done{0};
    auto body = [&]() {
      for (size_t i = next.fetch_add(1); i < n; i = next.fetch_add(1)) fn(i);
      done.fetch_add(1);
    };
    {
      std::lock_guard<std::mutex> lk(mu_);
      job_ = body;
      active_ = threads - 1;
      ++generation_;
    }
    cv_.notify_all();
    body();
    std::unique_lock<std::mutex> lk(mu_);
    done_cv_.wait(lk, [&] { return done.load() == threads; });
    job_ = nullptr;
  }

 private:
  CopyPool() {
    unsigned hw = std::thread::hardware_concurrency();
    unsigned n = std::max(1u, std::min(hw ? hw : 4u, 16u)) - 1;
    for (unsigned i = 0; i < n; ++i) workers_.emplace_back([this, i] { loop(i); });
  }
  static std::mutex& global_mu() {
    static std::mutex* mu = new std::mutex();  // never destroyed (see acquire)
    return *mu;
  }
  static std::shared_ptr<CopyPool>& global() {
    static std::shared_ptr<CopyPool>* inst = new std::shared_ptr<CopyPool>();  // never destroyed
    return *inst;
  }
  void loop(unsigned index) {
    sh::name_thread("sh-copy");
    running_.fetch_add(1);
    uint64_t seen = 0;
    for (;;) {
      std::function<void()> job;
      {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, [&] { return stop_ || generation_ != seen; });
        if (stop_) break;
        seen = generation_;
        if (index >= active_ || !job_) continue;
        job = job_;
      }
      job();
      std::lock_guard<std::mutex> lk(mu_);
      done_cv_.notify_all();
    }
    running_.fetch_sub(1);
  }

  std::vector<std::thread> workers_;
  std::mutex mu_, run_mu_;
  std::condition_variable cv_, done_cv_;
  std::function<void()> job_;
  unsigned active_ = 0;
  uint64_t generation_ = 0;
  bool stop_ = false;
  static std::atomic<int64_t> running_;
};

std::atomic<int64_t> CopyPool::running_{0};

constexpr size_t kCopyPiece = 8u << 20;  // 8 MiB pieces spread over the workers

}  // namespace

std::atomic<int64_t> sh::g_live[sh::kLiveKinds];

void sh::name_thread(const char* name) { (void)pthread_setname_np(pthread_self(), name); }

void sh::parallel_for(size_t n, unsigned threads, const std::function<void(size_t)>& fn) {
  if (n == 0) return;
  CopyPool::acquire()->parallel_for(n, threads, fn);
}

extern "C" int sh_shutdown(sh_live_counts* live) {
  sh::clear_error();
  // Dropping the global reference joins the copy threads here, or, when a parallel_for
  // is still running on another thread, as soon as it returns.
  CopyPool::take_global().reset();
  // The kernels' code is unloaded only when no engine that launches them is alive (loaders
  // launch the unpack and digests, save-back engines the comparisons, turbo engines both);
  // otherwise it stays loaded and the library holds it until the process ends.
  int status = SH_OK;
  const bool launchers = sh::g_live[sh::kLiveLoader].load() != 0 || sh::g_live[sh::kLiveSaveback].load() != 0 ||
                         sh::g_live[sh::kLiveTurbo].load() != 0;
  if (!launchers) {
    sh::noalloc_release();
    status = sh::unload_kernels();
  }
  if (live != nullptr) {
    live->pools = (uint64_t)sh::g_live[sh::kLivePool].load();
    live->loaders = (uint64_t)sh::g_live[sh::kLiveLoader].load();
    live->savebacks = (uint64_t)sh::g_live[sh::kLiveSaveback].load();
    live->turbos = (uint64_t)sh::g_live[sh::kLiveTurbo].load();
    live->vmms = (uint64_t)sh::g_live[sh::kLiveVmm].load();
    live->files = (uint64_t)sh::g_live[sh::kLiveFile].load();
    live->copy_threads = (uint64_t)CopyPool::running_threads();
    live->kernel_devices = (uint64_t)sh::kernels_loaded();
  }
  return status;
}

extern "C" int sh_host_copy_batch(const sh_copy_item* items, size_t n, int threads) {
  sh::clear_error();
  if (n > 0 && items == nullptr) return sh::fail(SH_ERR_INVALID, "sh_host_copy_batch: items is NULL");
  // Cut every item into pieces so that one large param spreads over all workers.
  std::vector<sh_copy_item> pieces;
  for (size_t i = 0; i < n; ++i) {
    const sh_copy_item& it = items[i];
    if (it.bytes == 0) continue;
    if (it.dst == nullptr || (it.src == nullptr && it.bytes > 0))
      return sh::fail(SH_ERR_INVALID, "sh_host_copy_batch: item %zu has a NULL pointer", i);
    for (uint64_t off = 0; off < it.bytes; off += kCopyPiece) {
      sh_copy_item p;
      p.dst = (uint8_t*)it.dst + off;
      p.src = (const uint8_t*)it.src + off;
      p.bytes = std::min<uint64_t>(kCopyPiece, it.bytes - off);
      pieces.push_back(p);
    }
  }
  sh::parallel_for(pieces.size(), threads > 0 ? (unsigned)threads : 1u, [&](size_t i) {
    std::memcpy(pieces[i].dst, pieces[i].src, pieces[i].bytes);
  });
  return SH_OK;
}
