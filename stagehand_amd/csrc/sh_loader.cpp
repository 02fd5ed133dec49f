// Block loader: a native worker that stages a block's parameter bytes into a
// pinned slab, copies the slab to the device on a copy stream and (for SquareQ
// or fp32 sources, or with chunk digests) runs the unpack / digest kernels once
// the copy has landed, all fenced by HIP events.
//
// This replaces the synchronous host path of the reference's block loads:
//   _stage_block_to_host       src/stagehand/scheduler.py:953-1031 (pool.acquire,
//                              per-parameter host copy / cast / dequant into the slab)
//   AsyncTransferEngine.submit_h2d  src/stagehand/transfer.py:108-143 (copy stream + event)
//   AsyncTransferEngine.wait   src/stagehand/transfer.py:193-217 (host event sync)
//   _finalize_gpu_load's slab release  src/stagehand/scheduler.py:1120-1124
// and the turbo engine's prefetch of turbo_src/engine.rs:202-230 / 267-282.
//
// Pipeline per request (ticket):
//   caller thread : record `ready` event on the caller's stream (the block's
//                   destination buffer was allocated there), enqueue request.
//   worker thread : acquire slab (blocks while every slab is busy; fenced
//                   slabs come back as their H2D copies drain), gather the
//                   pieces into the slab with the multi-threaded host copy
//                   and read its file ranges (pread / O_DIRECT) on the same
//                   threads,
//                   copy stream: wait `ready`, H2D slab → staging (or → dst),
//                   record `copied`; release the slab after `copied`.
//                   Without post-copy work (no plan, no digest) `done` is
//                   recorded right there.
//   post-copy work: the plan's unpack and the chunk digests, then `done`, are
//                   queued by the first caller that needs them:
//                   sh_loader_stream_wait queues them on the caller's stream
//                   behind a device wait on `copied`; sh_loader_query,
//                   sh_loader_sync, sh_loader_release, sh_loader_ticket_times
//                   and sh_loader_destroy queue them on the loader's unpack
//                   stream once `copied` has completed (query only looks;
//                   the others wait on the host).
//   caller thread : sh_loader_stream_wait(ticket, compute stream) makes the
//                   compute stream wait for the load without blocking the host.
// No stream of the loader therefore holds a device wait for a copy that is
// still queued. HIP maps its streams onto a few hardware queues
// (GPU_MAX_HW_QUEUES, 4 by default) and work of two streams that share one
// runs in the order it was queued: a wait for the next block's copy, queued
// on a loader stream that shares its hardware queue with the compute stream,
// held back every kernel queued behind it until that copy landed.
// The worker owns the host-side staging, so the Python hook thread never
// copies weight bytes and never waits for a copy to finish. When it starts a
// ticket, the buffered file ranges of that ticket and of the one queued behind
// it go to an advisor thread that asks the kernel to read them ahead
// (POSIX_FADV_WILLNEED): the whole range is queued as large reads at once, and
// the next block is already being read while the current one is staged.

#include <fcntl.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <condition_variable>
#include <cstring>
#include <deque>
#include <mutex>
#include <new>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "sh_internal.h"
#include "stagehand_native.h"

namespace {

enum class TicketState { Queued, Issued, Failed };

struct Ticket {
  TicketState state = TicketState::Queued;
  hipEvent_t ready = nullptr;   // recorded on the caller's stream at submit
  hipEvent_t copied = nullptr;  // H2D of the slab finished
  hipEvent_t done = nullptr;    // destination fully written
  hipEvent_t start = nullptr;   // timing only: copy stream reached this load
  int status = SH_OK;
  std::string error;
  // request
  std::vector<sh_copy_item> pieces;
  std::vector<sh_file_range> ranges;
  std::vector<sh_copy_item> dma;  // pinned sources copied straight to the device
  hipEvent_t wait_event = nullptr;
  sh_saveback* saveback = nullptr;  // save-back ticket waited for on the host before any copy
  uint64_t saveback_ticket = 0;
  bool advised = false;
  uint64_t src_bytes = 0;
  const sh_plan* plan = nullptr;
  void* staging = nullptr;
  uint64_t staging_bytes = 0;
  void* dst = nullptr;
  uint64_t dst_bytes = 0;
  int64_t scale_off = -1;
  int64_t zp_off = -1;
  uint64_t n_scale = 0;
  int copy_threads = 1;
  void* image = nullptr;
  uint64_t* digest = nullptr;  // chunk digests of dst once written (sh_block_digest)
  uint64_t digest_bytes = 0;
  uint32_t digest_chunk = 0;
  // the plan's unpack and the digests (then `done`) are still to be queued (launch_post)
  bool post_pending = false;
};

}  // namespace

struct sh_loader {
  sh::Live<sh::kLiveLoader> live;
  sh_pool* pool = nullptr;
  uint64_t slab_bytes = 0;
  int device = 0;
  int copy_threads = 1;
  hipStream_t copy_stream = nullptr;
  hipStream_t unpack_stream = nullptr;
  std::mutex mu;
  std::condition_variable cv;       // worker wakeup
  std::condition_variable issued_cv;  // ticket state changes
  std::deque<uint64_t> queue;
  std::unordered_map<uint64_t, Ticket> tickets;
  std::vector<hipEvent_t> spare_events;
  // image → event recorded after the last H2D that read it (worker thread only)
  std::unordered_map<void*, hipEvent_t> image_fence;
  uint64_t next_ticket = 1;
  bool stop = false;
  bool timing = false;  // copied/done/start are timing events
  std::vector<hipEvent_t> spare_timing_events;
  std::thread worker;
  // read-ahead advice: (fd, offset, bytes) handed to the advisor thread
  struct Advice {
    int fd;
    uint64_t off, bytes;
  };
  std::mutex advice_mu;
  std::condition_variable advice_cv;
  std::deque<Advice> advice;
  bool advice_stop = false;
  std::thread advisor;
};

extern "C" int sh_unpack(const sh_plan* plan, const void* src, size_t src_bytes, const float* scales,
                         const float* zero_points, size_t n_scale, void* dst, size_t dst_bytes, void* stream);

namespace {

hipError_t take_event(sh_loader* L, hipEvent_t* ev, bool timing = false) {
  std::vector<hipEvent_t>& spares = timing ? L->spare_timing_events : L->spare_events;
  if (!spares.empty()) {
    *ev = spares.back();
    spares.pop_back();
    return hipSuccess;
  }
  return hipEventCreateWithFlags(ev, timing ? hipEventDefault : hipEventDisableTiming);
}

void give_events(sh_loader* L, Ticket& t) {
  if (t.ready) L->spare_events.push_back(t.ready);
  const bool timed = t.start != nullptr;
  for (hipEvent_t* ev : {&t.copied, &t.done}) {
    if (*ev) (timed ? L->spare_timing_events : L->spare_events).push_back(*ev);
    *ev = nullptr;
  }
  if (t.start) L->spare_timing_events.push_back(t.start);
  t.ready = t.start = nullptr;
}

// Executes one request on the worker thread. Returns SH_OK or an error status
// with `err` describing it. Runs without the loader lock held.
int run_request(sh_loader* L, Ticket& t, std::string& err) {
  auto hip_fail = [&](hipError_t e, const char* what) {
    char buf[256];
    snprintf(buf, sizeof(buf), "HIP error %d (%s) in %s", (int)e, hipGetErrorString(e), what);
    err = buf;
    return SH_ERR_HIP;
  };
  hipError_t e = hipSetDevice(L->device);
  if (e != hipSuccess) return hip_fail(e, "hipSetDevice");

  // The source streams through the pool one slab-sized chunk at a time: gather
  // the chunk's part of every piece into a slab, H2D it, release the slab
  // after the copy. A block may therefore be larger than one slab; with two
  // or more slabs the gather of chunk k+1 overlaps the H2D of chunk k.
  void* h2d_dst = t.plan ? t.staging : t.dst;
  if (t.saveback != nullptr) {
    // the save-back that wrote pinned sources of this load runs on an SDMA engine: wait on the host
    int st = sh_saveback_wait(t.saveback, t.saveback_ticket);
    if (st != SH_OK) {
      err = sh_last_error();
      return st;
    }
  }
  e = hipStreamWaitEvent(L->copy_stream, t.ready, 0);
  if (e != hipSuccess) return hip_fail(e, "hipStreamWaitEvent(ready)");
  if (t.wait_event != nullptr) {
    e = hipStreamWaitEvent(L->copy_stream, t.wait_event, 0);
    if (e != hipSuccess) return hip_fail(e, "hipStreamWaitEvent(wait_event)");
  }
  if (t.start != nullptr) {
    e = hipEventRecord(t.start, L->copy_stream);
    if (e != hipSuccess) return hip_fail(e, "hipEventRecord(start)");
  }
  if (t.image != nullptr) {
    // Pinned source image: refresh the given pieces and ranges, then one DMA straight from it.
    if (!t.pieces.empty() || !t.ranges.empty() || !t.dma.empty()) {
      auto f = L->image_fence.find(t.image);
      if (f != L->image_fence.end()) {
        e = hipEventSynchronize(f->second);
        if (e != hipSuccess) return hip_fail(e, "hipEventSynchronize(image fence)");
      }
      if (!t.dma.empty() && t.wait_event != nullptr) {
        // the host copies the dma sources into the image: they must be final
        e = hipEventSynchronize(t.wait_event);
        if (e != hipSuccess) return hip_fail(e, "hipEventSynchronize(wait_event)");
      }
      std::vector<sh::IoPiece> io;
      for (const sh_copy_item& p : t.pieces)
        sh::append_copy(io, (uint8_t*)t.image + (uintptr_t)p.dst, p.src, p.bytes);
      for (const sh_copy_item& p : t.dma)
        sh::append_copy(io, (uint8_t*)t.image + (uintptr_t)p.dst, p.src, p.bytes);
      for (const sh_file_range& r : t.ranges)
        sh::append_read(io, r.file, r.file_off, r.bytes, (uint8_t*)t.image + r.dst);
      int st = sh::run_io(io, t.copy_threads);
      if (st != SH_OK) {
        err = sh_last_error();
        return st;
      }
    }
    if (t.src_bytes > 0) {
      e = hipMemcpyAsync(h2d_dst, t.image, t.src_bytes, hipMemcpyHostToDevice, L->copy_stream);
      if (e != hipSuccess) return hip_fail(e, "image H2D copy");
    }
    hipEvent_t fence = nullptr;
    auto f = L->image_fence.find(t.image);
    if (f != L->image_fence.end()) {
      fence = f->second;
    } else {
      e = hipEventCreateWithFlags(&fence, hipEventDisableTiming);
      if (e != hipSuccess) return hip_fail(e, "hipEventCreateWithFlags(image fence)");
      L->image_fence[t.image] = fence;
    }
    e = hipEventRecord(fence, L->copy_stream);
    if (e != hipSuccess) return hip_fail(e, "hipEventRecord(image fence)");
  }
  std::vector<sh::IoPiece> io;
  for (uint64_t c0 = 0; t.image == nullptr && c0 < t.src_bytes; c0 += L->slab_bytes) {
    const uint64_t c1 = std::min<uint64_t>(t.src_bytes, c0 + L->slab_bytes);
    if (!t.dma.empty()) {
      // only the regions of gathered pieces and ranges go through slabs
      bool any = false;
      for (const sh_copy_item& p : t.pieces)
        any = any || ((uint64_t)(uintptr_t)p.dst < c1 && (uint64_t)(uintptr_t)p.dst + p.bytes > c0 && p.bytes > 0);
      for (const sh_file_range& r : t.ranges) any = any || (r.dst < c1 && r.dst + r.bytes > c0 && r.bytes > 0);
      if (!any) continue;
    }
    uint32_t slab = 0;
    double waited = 0;
    int st = sh_pool_acquire(L->pool, -1, &slab, &waited);
    if (st != SH_OK) {
      err = sh_last_error();
      return st;
    }
    void* slab_ptr = nullptr;
    sh_pool_slab_ptr(L->pool, slab, &slab_ptr);
    io.clear();
    for (const sh_copy_item& p : t.pieces) {
      const uint64_t p0 = (uint64_t)(uintptr_t)p.dst, p1 = p0 + p.bytes;
      const uint64_t a = std::max(p0, c0), b = std::min(p1, c1);
      if (a < b) sh::append_copy(io, (uint8_t*)slab_ptr + (a - c0), (const uint8_t*)p.src + (a - p0), b - a);
    }
    for (const sh_file_range& r : t.ranges) {
      const uint64_t r0 = r.dst, r1 = r0 + r.bytes;
      const uint64_t a = std::max(r0, c0), b = std::min(r1, c1);
      if (a < b) sh::append_read(io, r.file, r.file_off + (a - r0), b - a, (uint8_t*)slab_ptr + (a - c0));
    }
    st = sh::run_io(io, t.copy_threads);
    if (st != SH_OK) {
      err = sh_last_error();
      sh_pool_release(L->pool, slab);
      return st;
    }
    if (t.dma.empty()) {
      e = hipMemcpyAsync((uint8_t*)h2d_dst + c0, slab_ptr, c1 - c0, hipMemcpyHostToDevice, L->copy_stream);
    } else {
      // the dma pieces write their own regions: send only what was gathered here
      std::vector<std::pair<uint64_t, uint64_t>> iv;
      for (const sh::IoPiece& p : io) {
        const uint64_t a = (uint64_t)(p.dst - (uint8_t*)slab_ptr);
        iv.emplace_back(a, a + p.bytes);
      }
      std::sort(iv.begin(), iv.end());
      e = hipSuccess;
      for (size_t i = 0; i < iv.size() && e == hipSuccess;) {
        uint64_t a = iv[i].first, b = iv[i].second;
        for (++i; i < iv.size() && iv[i].first <= b; ++i) b = std::max(b, iv[i].second);
        e = hipMemcpyAsync((uint8_t*)h2d_dst + c0 + a, (uint8_t*)slab_ptr + a, b - a, hipMemcpyHostToDevice,
                           L->copy_stream);
      }
    }
    if (e != hipSuccess) {
      (void)hipStreamSynchronize(L->copy_stream);
      sh_pool_release(L->pool, slab);
      return hip_fail(e, "staging H2D copy");
    }
    st = sh_pool_release_after(L->pool, slab, L->copy_stream);
    if (st != SH_OK) {
      err = sh_last_error();
      return st;
    }
  }
  if (t.image == nullptr) {
    for (const sh_copy_item& p : t.dma) {
      if (p.bytes == 0) continue;
      e = hipMemcpyAsync((uint8_t*)h2d_dst + (uintptr_t)p.dst, p.src, p.bytes, hipMemcpyHostToDevice, L->copy_stream);
      if (e != hipSuccess) return hip_fail(e, "pinned-source H2D copy");
    }
  }
  e = hipEventRecord(t.copied, L->copy_stream);
  if (e != hipSuccess) return hip_fail(e, "hipEventRecord(copied)");
  if (!t.post_pending) {
    e = hipEventRecord(t.done, L->copy_stream);
    if (e != hipSuccess) return hip_fail(e, "hipEventRecord(done)");
  }
  return SH_OK;
}

// Queues ticket `t`'s post-copy work (the plan's unpack, the chunk digests) on `stream` behind a
// device wait on `copied`, and records `done` after it. Called with L->mu held, once per ticket,
// after the worker has issued it. On failure the ticket fails, and `done` still marks the end of
// whatever was queued.
int launch_post(sh_loader* L, Ticket& t, hipStream_t stream, const char* who) {
  t.post_pending = false;
  int prev = -1;
  (void)hipGetDevice(&prev);
  hipError_t e = prev == L->device ? hipSuccess : hipSetDevice(L->device);
  int st = SH_OK;
  if (e == hipSuccess) e = hipStreamWaitEvent(stream, t.copied, 0);
  if (e != hipSuccess) {
    st = sh::fail(SH_ERR_HIP, "%s: ordering the unpack after the copy: HIP error %d (%s)", who, (int)e,
                  hipGetErrorString(e));
  }
  if (st == SH_OK && t.plan != nullptr) {
    const uint8_t* stg = (const uint8_t*)t.staging;
    const float* scales = t.scale_off >= 0 ? (const float*)(stg + t.scale_off) : nullptr;
    const float* zps = t.zp_off >= 0 ? (const float*)(stg + t.zp_off) : nullptr;
    st = sh_unpack(t.plan, t.staging, t.staging_bytes, scales, zps, t.n_scale, t.dst, t.dst_bytes, stream);
  }
  if (st == SH_OK && t.digest != nullptr)
    st = sh::launch_block_digest(t.dst, t.digest_bytes, t.digest_chunk, t.digest, stream);
  e = hipEventRecord(t.done, stream);
  if (st == SH_OK && e != hipSuccess)
    st = sh::fail(SH_ERR_HIP, "%s: hipEventRecord(done): HIP error %d (%s)", who, (int)e, hipGetErrorString(e));
  if (prev >= 0 && prev != L->device) (void)hipSetDevice(prev);
  if (st != SH_OK) {
    t.status = st;
    t.error = sh_last_error();
    t.state = TicketState::Failed;
    L->issued_cv.notify_all();
  }
  return st;
}

// Queues POSIX_FADV_WILLNEED for the buffered file ranges of `t` (once per
// ticket). One advice call per range makes the kernel queue the whole range's
// reads at once, in large requests, where the copy threads' preads alone would
// read a cold file one small read-ahead window at a time. Called with L->mu held.
void advise(sh_loader* L, Ticket& t) {
  if (t.advised || t.ranges.empty()) return;
  t.advised = true;
  std::lock_guard<std::mutex> ag(L->advice_mu);
  for (const sh_file_range& r : t.ranges) {
    const int fd = sh::advice_fd(r.file);
    if (fd >= 0 && r.bytes > 0) L->advice.push_back({fd, r.file_off, r.bytes});
  }
  L->advice_cv.notify_one();
}

void worker_loop(sh_loader* L) {
  sh::name_thread("sh-loader");
  for (;;) {
    uint64_t id = 0;
    Ticket* t = nullptr;
    {
      std::unique_lock<std::mutex> lk(L->mu);
      L->cv.wait(lk, [&] { return L->stop || !L->queue.empty(); });
      if (L->queue.empty()) return;  // stop requested and drained
      id = L->queue.front();
      L->queue.pop_front();
      t = &L->tickets.at(id);  // unordered_map references stay valid across inserts
      // read-ahead advice for this ticket's files, then the next one's (their files are
      // open until the tickets are issued: take the descriptors now)
      advise(L, *t);
      if (!L->queue.empty()) advise(L, L->tickets.at(L->queue.front()));
    }
    std::string err;
    const int st = run_request(L, *t, err);
    if (st != SH_OK) {
      // Chunks copied before the failure may still be landing in the destination: mark their
      // end so that releasing the ticket waits for them (no post-copy work was queued).
      (void)hipEventRecord(t->copied, L->copy_stream);
      (void)hipEventRecord(t->done, L->copy_stream);
    }
    {
      std::lock_guard<std::mutex> lk(L->mu);
      t->status = st;
      t->error = err;
      t->state = st == SH_OK ? TicketState::Issued : TicketState::Failed;
      if (st != SH_OK) t->post_pending = false;
      t->pieces.clear();
      t->pieces.shrink_to_fit();
      t->ranges.clear();
      t->ranges.shrink_to_fit();
      t->dma.clear();
      t->dma.shrink_to_fit();
      t->wait_event = nullptr;
      t->saveback = nullptr;
    }
    L->issued_cv.notify_all();
  }
}

// Gives read-ahead advice off the worker thread: posix_fadvise(WILLNEED) starts
// the reads but may block while it queues them. The descriptors were taken
// while their files were known to be open; advice on a descriptor that has
// since been closed or reused is at worst a wasted hint.
void advisor_loop(sh_loader* L) {
  sh::name_thread("sh-advisor");
  for (;;) {
    sh_loader::Advice a;
    {
      std::unique_lock<std::mutex> lk(L->advice_mu);
      L->advice_cv.wait(lk, [&] { return L->advice_stop || !L->advice.empty(); });
      if (L->advice_stop) return;
      a = L->advice.front();
      L->advice.pop_front();
    }
    (void)::posix_fadvise(a.fd, (off_t)a.off, (off_t)a.bytes, POSIX_FADV_WILLNEED);
  }
}

// Waits (caller thread) until the worker has issued or failed ticket `id`.
// Returns SH_OK with *out set, or an error status.
int wait_issued(sh_loader* L, uint64_t id, std::unique_lock<std::mutex>& lk, Ticket** out, const char* who) {
  auto it = L->tickets.find(id);
  if (it == L->tickets.end()) return sh::fail(SH_ERR_INVALID, "%s: unknown ticket %llu", who, (unsigned long long)id);
  L->issued_cv.wait(lk, [&] { return it->second.state != TicketState::Queued; });
  if (it->second.state == TicketState::Failed)
    return sh::fail(it->second.status == SH_OK ? SH_ERR_HIP : it->second.status, "%s: load failed: %s", who,
                    it->second.error.c_str());
  *out = &it->second;
  return SH_OK;
}

// Queues ticket `id`'s post-copy work on the unpack stream if no caller has queued it yet, once
// its copy has landed (the host waits for that). Called without L->mu held. SH_OK also for a
// ticket that has failed (nothing is left to queue for it).
int finish_post(sh_loader* L, uint64_t id, const char* who) {
  hipEvent_t copied = nullptr;
  {
    std::unique_lock<std::mutex> lk(L->mu);
    auto it = L->tickets.find(id);
    if (it == L->tickets.end()) return sh::fail(SH_ERR_INVALID, "%s: unknown ticket %llu", who, (unsigned long long)id);
    L->issued_cv.wait(lk, [&] { return it->second.state != TicketState::Queued; });
    if (!it->second.post_pending) return SH_OK;
    copied = it->second.copied;
  }
  const hipError_t e = hipEventSynchronize(copied);
  if (e != hipSuccess)
    return sh::fail(SH_ERR_HIP, "%s: waiting for the copy: HIP error %d (%s)", who, (int)e, hipGetErrorString(e));
  std::lock_guard<std::mutex> lk(L->mu);
  auto it = L->tickets.find(id);
  if (it == L->tickets.end() || !it->second.post_pending) return SH_OK;
  return launch_post(L, it->second, L->unpack_stream, who);
}

}  // namespace

extern "C" int sh_loader_create(sh_pool* pool, int copy_threads, sh_loader** out) {
  sh::clear_error();
  if (pool == nullptr || out == nullptr) return sh::fail(SH_ERR_INVALID, "sh_loader_create: NULL argument");
  *out = nullptr;
  sh_loader* L = new (std::nothrow) sh_loader();
  if (L == nullptr) return sh::fail(SH_ERR_OOM, "sh_loader_create: out of host memory");
  L->pool = pool;
  L->copy_threads = copy_threads > 0 ? copy_threads : 1;
  sh_pool_stats ps{};
  if (int st = sh_pool_get_stats(pool, &ps)) {
    delete L;
    return st;
  }
  L->slab_bytes = ps.slab_bytes;
  hipError_t e = hipGetDevice(&L->device);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&L->copy_stream, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&L->unpack_stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    if (L->copy_stream) (void)hipStreamDestroy(L->copy_stream);
    if (L->unpack_stream) (void)hipStreamDestroy(L->unpack_stream);
    delete L;
    return sh::fail(SH_ERR_HIP, "sh_loader_create: HIP error %d (%s)", (int)e, hipGetErrorString(e));
  }
  L->worker = std::thread(worker_loop, L);
  L->advisor = std::thread(advisor_loop, L);
  *out = L;
  return SH_OK;
}

extern "C" int sh_loader_destroy(sh_loader* L) {
  sh::clear_error();
  if (L == nullptr) return SH_OK;
  {
    std::lock_guard<std::mutex> lk(L->mu);
    L->stop = true;
  }
  L->cv.notify_all();
  if (L->worker.joinable()) L->worker.join();
  {
    std::lock_guard<std::mutex> ag(L->advice_mu);
    L->advice_stop = true;
  }
  L->advice_cv.notify_all();
  if (L->advisor.joinable()) L->advisor.join();
  // tickets never waited for still get their post-copy work, as they would have on release
  std::vector<uint64_t> pending;
  for (const auto& kv : L->tickets)
    if (kv.second.post_pending) pending.push_back(kv.first);
  for (uint64_t id : pending) (void)finish_post(L, id, "sh_loader_destroy");
  (void)hipStreamSynchronize(L->copy_stream);
  (void)hipStreamSynchronize(L->unpack_stream);
  for (auto& kv : L->tickets) give_events(L, kv.second);
  for (hipEvent_t ev : L->spare_events) (void)hipEventDestroy(ev);
  for (hipEvent_t ev : L->spare_timing_events) (void)hipEventDestroy(ev);
  for (auto& kv : L->image_fence) (void)hipEventDestroy(kv.second);
  (void)hipStreamDestroy(L->copy_stream);
  (void)hipStreamDestroy(L->unpack_stream);
  delete L;
  return SH_OK;
}

extern "C" int sh_loader_streams(sh_loader* L, void** copy_stream, void** unpack_stream) {
  sh::clear_error();
  if (L == nullptr) return sh::fail(SH_ERR_INVALID, "sh_loader_streams: loader is NULL");
  if (copy_stream) *copy_stream = (void*)L->copy_stream;
  if (unpack_stream) *unpack_stream = (void*)L->unpack_stream;
  return SH_OK;
}

extern "C" int sh_loader_submit(sh_loader* L, const sh_load_request* req, void* wait_stream, uint64_t* ticket) {
  sh::clear_error();
  if (L == nullptr || req == nullptr || ticket == nullptr) return sh::fail(SH_ERR_INVALID, "sh_loader_submit: NULL argument");
  if (req->n_pieces > 0 && req->pieces == nullptr) return sh::fail(SH_ERR_INVALID, "sh_loader_submit: pieces is NULL");
  if (req->dst == nullptr && req->dst_bytes > 0) return sh::fail(SH_ERR_INVALID, "sh_loader_submit: dst is NULL");
  uint64_t need = 0;
  for (uint64_t i = 0; i < req->n_pieces; ++i) {
    const sh_copy_item& p = req->pieces[i];
    const uint64_t end = (uint64_t)(uintptr_t)p.dst + p.bytes;
    if (end < p.bytes) return sh::fail(SH_ERR_INVALID, "sh_loader_submit: piece %llu overflows", (unsigned long long)i);
    if (p.bytes > 0 && p.src == nullptr) return sh::fail(SH_ERR_INVALID, "sh_loader_submit: piece %llu has no source", (unsigned long long)i);
    need = need > end ? need : end;
  }
  if (req->n_ranges > 0 && req->ranges == nullptr) return sh::fail(SH_ERR_INVALID, "sh_loader_submit: ranges is NULL");
  for (uint64_t i = 0; i < req->n_ranges; ++i) {
    const sh_file_range& r = req->ranges[i];
    if (int st = sh::check_range(r.file, r.file_off, r.bytes, "sh_loader_submit")) return st;
    const uint64_t end = r.dst + r.bytes;
    if (end < r.bytes) return sh::fail(SH_ERR_INVALID, "sh_loader_submit: range %llu overflows", (unsigned long long)i);
    need = need > end ? need : end;
  }
  if (req->n_dma > 0 && req->dma == nullptr) return sh::fail(SH_ERR_INVALID, "sh_loader_submit: dma is NULL");
  for (uint64_t i = 0; i < req->n_dma; ++i) {
    const sh_copy_item& p = req->dma[i];
    const uint64_t end = (uint64_t)(uintptr_t)p.dst + p.bytes;
    if (end < p.bytes) return sh::fail(SH_ERR_INVALID, "sh_loader_submit: dma piece %llu overflows", (unsigned long long)i);
    if (p.bytes > 0 && p.src == nullptr)
      return sh::fail(SH_ERR_INVALID, "sh_loader_submit: dma piece %llu has no source", (unsigned long long)i);
    need = need > end ? need : end;
  }
  if (need > req->src_bytes) return sh::fail(SH_ERR_INVALID, "sh_loader_submit: pieces end at %llu, past src_bytes %llu",
                                             (unsigned long long)need, (unsigned long long)req->src_bytes);
  if (req->plan != nullptr) {
    sh_plan_info info{};
    sh_plan_get_info(req->plan, &info);
    if (req->staging == nullptr || req->staging_bytes < req->src_bytes)
      return sh::fail(SH_ERR_INVALID, "sh_loader_submit: device staging buffer smaller than the source");
    if (info.src_extent > req->src_bytes)
      return sh::fail(SH_ERR_INVALID, "sh_loader_submit: plan reads %llu source bytes, only %llu are sent",
                      (unsigned long long)info.src_extent, (unsigned long long)req->src_bytes);
    if (req->dst_bytes < info.dst_extent)
      return sh::fail(SH_ERR_INVALID, "sh_loader_submit: destination smaller than the plan's extent");
    const bool has_i8 = (info.kind_mask & ((1u << SH_KIND_I8_ROWSCALE_BF16) | (1u << SH_KIND_I8_ROWSCALE_F32))) != 0;
    if (has_i8) {
      if (req->scale_off < 0 || (req->scale_off % 4) != 0 ||
          (uint64_t)req->scale_off + 4 * req->n_scale > req->src_bytes || req->n_scale < info.scale_extent)
        return sh::fail(SH_ERR_INVALID, "sh_loader_submit: scales are not inside the source or too few");
      if (req->zp_off >= 0 && ((req->zp_off % 4) != 0 || (uint64_t)req->zp_off + 4 * req->n_scale > req->src_bytes))
        return sh::fail(SH_ERR_INVALID, "sh_loader_submit: zero points are not inside the source");
    }
  } else if (req->dst_bytes < req->src_bytes) {
    return sh::fail(SH_ERR_INVALID, "sh_loader_submit: destination smaller than the source bytes");
  }
  if (req->digest != nullptr) {
    if (req->digest_bytes > req->dst_bytes)
      return sh::fail(SH_ERR_INVALID, "sh_loader_submit: digest of %llu bytes past the destination's %llu",
                      (unsigned long long)req->digest_bytes, (unsigned long long)req->dst_bytes);
    if (req->digest_chunk == 0 || req->digest_chunk % 16 != 0)
      return sh::fail(SH_ERR_INVALID, "sh_loader_submit: digest_chunk %u is not a positive multiple of 16",
                      req->digest_chunk);
  }

  std::lock_guard<std::mutex> lk(L->mu);
  const uint64_t id = L->next_ticket++;
  Ticket& t = L->tickets[id];
  hipError_t e = take_event(L, &t.ready);
  if (e == hipSuccess) e = take_event(L, &t.copied, L->timing);
  if (e == hipSuccess) e = take_event(L, &t.done, L->timing);
  if (e == hipSuccess && L->timing) e = take_event(L, &t.start, true);
  if (e == hipSuccess) e = hipEventRecord(t.ready, (hipStream_t)wait_stream);
  if (e != hipSuccess) {
    give_events(L, t);
    L->tickets.erase(id);
    return sh::fail(SH_ERR_HIP, "sh_loader_submit: HIP error %d (%s)", (int)e, hipGetErrorString(e));
  }
  t.pieces.assign(req->pieces, req->pieces + req->n_pieces);
  if (req->n_ranges > 0) t.ranges.assign(req->ranges, req->ranges + req->n_ranges);
  if (req->n_dma > 0) t.dma.assign(req->dma, req->dma + req->n_dma);
  t.wait_event = (hipEvent_t)req->wait_event;
  t.saveback = req->saveback;
  t.saveback_ticket = req->saveback_ticket;
  t.src_bytes = req->src_bytes;
  t.plan = req->plan;
  t.staging = req->staging;
  t.staging_bytes = req->staging_bytes;
  t.dst = req->dst;
  t.dst_bytes = req->dst_bytes;
  t.scale_off = req->scale_off;
  t.zp_off = req->zp_off;
  t.n_scale = req->n_scale;
  t.copy_threads = req->copy_threads > 0 ? req->copy_threads : L->copy_threads;
  t.image = req->image;
  t.digest = req->digest;
  t.digest_bytes = req->digest_bytes;
  t.digest_chunk = req->digest_chunk;
  t.post_pending = t.plan != nullptr || t.digest != nullptr;
  L->queue.push_back(id);
  *ticket = id;
  L->cv.notify_one();
  return SH_OK;
}

extern "C" int sh_loader_query(sh_loader* L, uint64_t ticket) {
  sh::clear_error();
  if (L == nullptr) return sh::fail(SH_ERR_INVALID, "sh_loader_query: loader is NULL");
  std::lock_guard<std::mutex> lk(L->mu);
  auto it = L->tickets.find(ticket);
  if (it == L->tickets.end()) return sh::fail(SH_ERR_INVALID, "sh_loader_query: unknown ticket %llu", (unsigned long long)ticket);
  Ticket& t = it->second;
  if (t.state == TicketState::Queued) return SH_ERR_NOT_READY;
  if (t.state == TicketState::Failed) return sh::fail(t.status, "sh_loader_query: load failed: %s", t.error.c_str());
  if (t.post_pending) {
    // the copy has landed: queue the post-copy work on the unpack stream, with nothing to wait for
    const hipError_t c = hipEventQuery(t.copied);
    if (c == hipErrorNotReady) return SH_ERR_NOT_READY;
    SH_HIP(c);
    if (int st = launch_post(L, t, L->unpack_stream, "sh_loader_query")) return st;
  }
  const hipError_t e = hipEventQuery(t.done);
  if (e == hipErrorNotReady) return SH_ERR_NOT_READY;
  SH_HIP(e);
  return SH_OK;
}

extern "C" int sh_loader_query_copy(sh_loader* L, uint64_t ticket) {
  sh::clear_error();
  if (L == nullptr) return sh::fail(SH_ERR_INVALID, "sh_loader_query_copy: loader is NULL");
  std::lock_guard<std::mutex> lk(L->mu);
  auto it = L->tickets.find(ticket);
  if (it == L->tickets.end())
    return sh::fail(SH_ERR_INVALID, "sh_loader_query_copy: unknown ticket %llu", (unsigned long long)ticket);
  Ticket& t = it->second;
  if (t.state == TicketState::Queued) return SH_ERR_NOT_READY;
  if (t.state == TicketState::Failed) return sh::fail(t.status, "sh_loader_query_copy: load failed: %s", t.error.c_str());
  const hipError_t e = hipEventQuery(t.copied);
  if (e == hipErrorNotReady) return SH_ERR_NOT_READY;
  SH_HIP(e);
  return SH_OK;
}

extern "C" int sh_loader_sync_copy(sh_loader* L, uint64_t ticket) {
  sh::clear_error();
  if (L == nullptr) return sh::fail(SH_ERR_INVALID, "sh_loader_sync_copy: loader is NULL");
  hipEvent_t copied = nullptr;
  {
    std::unique_lock<std::mutex> lk(L->mu);
    Ticket* t = nullptr;
    if (int st = wait_issued(L, ticket, lk, &t, "sh_loader_sync_copy")) return st;
    copied = t->copied;
  }
  SH_HIP(hipEventSynchronize(copied));
  return SH_OK;
}

extern "C" int sh_loader_stream_wait(sh_loader* L, uint64_t ticket, void* stream) {
  sh::clear_error();
  if (L == nullptr) return sh::fail(SH_ERR_INVALID, "sh_loader_stream_wait: loader is NULL");
  std::unique_lock<std::mutex> lk(L->mu);
  Ticket* t = nullptr;
  if (int st = wait_issued(L, ticket, lk, &t, "sh_loader_stream_wait")) return st;
  if (t->post_pending) return launch_post(L, *t, (hipStream_t)stream, "sh_loader_stream_wait");
  SH_HIP(hipStreamWaitEvent((hipStream_t)stream, t->done, 0));
  return SH_OK;
}

extern "C" int sh_loader_sync(sh_loader* L, uint64_t ticket) {
  sh::clear_error();
  if (L == nullptr) return sh::fail(SH_ERR_INVALID, "sh_loader_sync: loader is NULL");
  if (int st = finish_post(L, ticket, "sh_loader_sync")) return st;
  hipEvent_t done = nullptr;
  {
    std::unique_lock<std::mutex> lk(L->mu);
    Ticket* t = nullptr;
    if (int st = wait_issued(L, ticket, lk, &t, "sh_loader_sync")) return st;
    done = t->done;
  }
  SH_HIP(hipEventSynchronize(done));
  return SH_OK;
}

extern "C" int sh_loader_release(sh_loader* L, uint64_t ticket) {
  sh::clear_error();
  if (L == nullptr) return sh::fail(SH_ERR_INVALID, "sh_loader_release: loader is NULL");
  // a ticket nobody waited for still gets its post-copy work: the destination is written on return
  const int post = finish_post(L, ticket, "sh_loader_release");
  std::unique_lock<std::mutex> lk(L->mu);
  auto it = L->tickets.find(ticket);
  if (it == L->tickets.end()) return sh::fail(SH_ERR_INVALID, "sh_loader_release: unknown ticket %llu", (unsigned long long)ticket);
  // Never recycle events the worker may still record: wait until it is done with the ticket.
  L->issued_cv.wait(lk, [&] { return it->second.state != TicketState::Queued; });
  hipEvent_t done = it->second.done;
  lk.unlock();
  // Events go back to the spare list only once the device has passed them (a
  // failed ticket's events mark the copies queued before the failure).
  const hipError_t e = hipEventSynchronize(done);
  lk.lock();
  it = L->tickets.find(ticket);
  if (it != L->tickets.end()) {
    give_events(L, it->second);
    L->tickets.erase(it);
  }
  if (e != hipSuccess) return sh::fail(SH_ERR_HIP, "sh_loader_release: HIP error %d", (int)e);
  return post;
}

extern "C" int sh_loader_set_timing(sh_loader* L, int enable) {
  sh::clear_error();
  if (L == nullptr) return sh::fail(SH_ERR_INVALID, "sh_loader_set_timing: loader is NULL");
  std::lock_guard<std::mutex> lk(L->mu);
  L->timing = enable != 0;
  return SH_OK;
}

extern "C" int sh_loader_ticket_times(sh_loader* L, uint64_t ticket, void* ref_event, float* out3) {
  sh::clear_error();
  if (L == nullptr || ref_event == nullptr || out3 == nullptr)
    return sh::fail(SH_ERR_INVALID, "sh_loader_ticket_times: NULL argument");
  if (int st = finish_post(L, ticket, "sh_loader_ticket_times")) return st;
  hipEvent_t start = nullptr, copied = nullptr, done = nullptr;
  {
    std::unique_lock<std::mutex> lk(L->mu);
    Ticket* t = nullptr;
    if (int st = wait_issued(L, ticket, lk, &t, "sh_loader_ticket_times")) return st;
    if (t->start == nullptr) return sh::fail(SH_ERR_STATE, "sh_loader_ticket_times: ticket was submitted without timing");
    start = t->start;
    copied = t->copied;
    done = t->done;
  }
  SH_HIP(hipEventSynchronize(done));
  SH_HIP(hipEventElapsedTime(&out3[0], (hipEvent_t)ref_event, start));
  SH_HIP(hipEventElapsedTime(&out3[1], (hipEvent_t)ref_event, copied));
  SH_HIP(hipEventElapsedTime(&out3[2], (hipEvent_t)ref_event, done));
  return SH_OK;
}
