// Save-back copies (device -> pinned host) on a system DMA (SDMA) engine.
//
// Eviction with save-back copies a block's device bytes into host memory (the
// reference's `param.data.to("cpu")`, src/stagehand/scheduler.py:1216-1226 and
// 1348-1366). hipMemcpyAsync runs a pinned device-to-host copy as a kernel on
// the compute units; on MI355X the compute kernels that ran beside those copies
// in a streamed training step took many times their usual duration (a 740 MB
// block copy overlapping a GEMM, attention or elementwise kernel; a copy
// kernel limited to 16 workgroups still did it, a CU-masked copy stream
// helped little). The SDMA engines copy without the compute units, so the
// copies here go through the HSA runtime's hsa_amd_memory_async_copy, which
// uses them for transfers between a GPU agent and the CPU agent.
//
// Ordering: an HSA copy cannot wait for a HIP event on the device, so each
// submit records an event on the caller's stream and a worker thread waits
// for it on the host before it issues the copies (or, for
// sh_saveback_submit_after, waits for the caller's own events). Completion: each copy has an
// HSA signal of its own, initialised to 1, which the copy engine decrements. (HSA
// lets several copies share one signal initialised to their count, but the
// profiler's copy tracing replaces each copy's completion signal and forwards
// one completion per copy: with a shared signal it reported "bad original signal
// value" and completions that were never delivered.) Tickets complete in
// submission order: query and wait report a ticket done only when every live
// earlier ticket is, so a later ticket covers earlier copies as a later event on
// one stream would.
//
// Chunk save-backs (sh_saveback_submit_chunks): when the caller has digests of what
// the host buffer holds (sh_digest.hip), the submit queues their comparison with the
// device buffer on a stream the caller names, ordered after the caller's events, and
// the job's fence after it; the worker, once the fence has passed, reads the flags
// and copies back only the runs of chunks whose digests changed. Such a ticket's
// copies are decided by the worker: waiters wait until it has set them.

#include <hip/hip_runtime.h>
#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstdint>
#include <deque>
#include <map>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

#include "sh_internal.h"
#include "stagehand_native.h"

namespace {

// A ticket's state. Its signals and fence belong to the object and are destroyed with it,
// when the last reference drops: the queue's, the worker's, a waiter's snapshot or the
// engine's map entry. Releasing a ticket therefore never frees a signal that a waiter on a
// later ticket, or the worker, still holds.
struct Job {
  uint64_t id = 0;
  hipEvent_t fence = nullptr;  // none for a ticket without copies
  hipEvent_t order = nullptr;  // a chunk job's: the caller's stream, which its comparison waits for
  std::vector<hipEvent_t> after;  // the caller's events (sh_saveback_submit_after), not owned
  std::vector<sh_copy_item> items;
  std::vector<hsa_signal_t> done;  // done[k]: 1 until items[k] has been copied
  int status = SH_OK;  // set (under the engine lock) before a failure completes the signals
  std::string error;
  uint64_t copied = 0;  // bytes the items move
  // sh_saveback_submit_chunks: the worker picks the copies (items, done, copied) once the
  // fences have passed, then sets `issued`; until then waiters wait for it.
  bool chunked = false;
  std::vector<sh_chunk_region> regions;
  uint32_t chunk = 0;
  const uint64_t* digests = nullptr;
  uint8_t* changed = nullptr;
  bool issued = true;  // guarded by the engine lock

  Job() = default;
  Job(const Job&) = delete;
  Job& operator=(const Job&) = delete;
  ~Job() {
    for (hsa_signal_t s : done)
      if (s.handle != 0) hsa_signal_destroy(s);
    if (fence != nullptr) (void)hipEventDestroy(fence);
    if (order != nullptr) (void)hipEventDestroy(order);
  }
};

hsa_status_t find_cpu(hsa_agent_t agent, void* data) {
  hsa_device_type_t type;
  if (hsa_agent_get_info(agent, HSA_AGENT_INFO_DEVICE, &type) == HSA_STATUS_SUCCESS && type == HSA_DEVICE_TYPE_CPU) {
    *(hsa_agent_t*)data = agent;
    return HSA_STATUS_INFO_BREAK;
  }
  return HSA_STATUS_SUCCESS;
}

}  // namespace

struct sh_saveback {
  sh::Live<sh::kLiveSaveback> live;
  int device = 0;
  hsa_agent_t cpu{0}, gpu{0};
  std::mutex mu;
  std::condition_variable cv;
  std::deque<std::shared_ptr<Job>> queue;          // submitted, not yet issued by the worker
  std::map<uint64_t, std::shared_ptr<Job>> jobs;   // every live ticket, in submission order
  uint64_t next_id = 1;
  bool stop = false;
  std::atomic<bool> timing{false};  // read by the worker without the lock
  std::condition_variable issued_cv;  // a chunk job's copies were picked
  std::thread worker;
};

namespace {

// Records a failure, then completes the signals of the copies from `first` on, which were
// never issued (waiters read the status after the signals).
void fail_job(sh_saveback* sb, Job& j, int status, const std::string& what, size_t first) {
  {
    std::lock_guard<std::mutex> lk(sb->mu);
    j.status = status;
    j.error = what;
    j.issued = true;  // a chunk job that failed before its copies were picked has none
  }
  sb->issued_cv.notify_all();
  for (size_t k = first; k < j.done.size(); ++k) hsa_signal_subtract_screlease(j.done[k], 1);
}

// For a chunk job whose fence has passed (and with it the comparison of its digests, queued
// before the fence): sets the job's copies, one per run of changed chunks (every chunk without
// digests), with a signal each, and publishes them.
int pick_chunks(sh_saveback* sb, Job& j, std::string& err) {
  auto chunks_of = [&](uint64_t bytes) { return bytes / j.chunk + (bytes % j.chunk != 0 ? 1 : 0); };
  // the comparison ran on the device before the job's fence, which has passed
  std::vector<sh_copy_item> runs;
  const volatile uint8_t* changed = j.changed;
  for (const sh_chunk_region& r : j.regions) {
    const uint64_t n = chunks_of(r.bytes);
    const volatile uint8_t* f = j.digests != nullptr ? changed + r.first_chunk : nullptr;
    for (uint64_t c = 0; c < n;) {
      if (f != nullptr && f[c] == 0) {
        ++c;
        continue;
      }
      uint64_t c1 = c + 1;
      while (c1 < n && (f == nullptr || f[c1] != 0)) ++c1;
      const uint64_t b = c * j.chunk, e = c1 < n ? c1 * j.chunk : r.bytes;
      runs.push_back(sh_copy_item{(uint8_t*)r.host_dst + b, (const uint8_t*)r.dev_src + b, e - b});
      c = c1;
    }
  }
  std::vector<hsa_signal_t> sigs;
  for (size_t k = 0; k < runs.size(); ++k) {
    hsa_signal_t s{0};
    if (hsa_signal_create(1, 0, nullptr, &s) != HSA_STATUS_SUCCESS) {
      for (hsa_signal_t t : sigs) hsa_signal_destroy(t);
      err = "hsa_signal_create failed";
      return SH_ERR_HIP;
    }
    sigs.push_back(s);
  }
  {
    std::lock_guard<std::mutex> lk(sb->mu);
    j.copied = 0;
    for (const sh_copy_item& r : runs) j.copied += r.bytes;
    j.items = std::move(runs);
    j.done = std::move(sigs);
    j.issued = true;
  }
  sb->issued_cv.notify_all();
  return SH_OK;
}

void worker_loop(sh_saveback* sb) {
  sh::name_thread("sh-saveback");
  (void)hipSetDevice(sb->device);
  for (;;) {
    std::shared_ptr<Job> j;
    {
      std::unique_lock<std::mutex> lk(sb->mu);
      sb->cv.wait(lk, [&] { return sb->stop || !sb->queue.empty(); });
      if (sb->queue.empty()) return;  // stop requested and nothing left to issue
      j = sb->queue.front();
      sb->queue.pop_front();
    }
    hipError_t e = j->fence != nullptr ? hipEventSynchronize(j->fence) : hipSuccess;
    for (size_t k = 0; e == hipSuccess && k < j->after.size(); ++k) e = hipEventSynchronize(j->after[k]);
    if (e != hipSuccess) {
      fail_job(sb, *j, SH_ERR_HIP, std::string("hipEventSynchronize(save-back fence): ") + hipGetErrorString(e), 0);
      continue;
    }
    if (j->chunked) {
      std::string err;
      const int st = pick_chunks(sb, *j, err);
      if (st != SH_OK) {
        fail_job(sb, *j, st, err, 0);
        continue;
      }
    }
    for (size_t k = 0; k < j->items.size(); ++k) {
      const sh_copy_item& it = j->items[k];
      hsa_status_t s = hsa_amd_memory_async_copy(it.dst, sb->cpu, it.src, sb->gpu, it.bytes, 0, nullptr, j->done[k]);
      if (s != HSA_STATUS_SUCCESS) {
        const char* msg = nullptr;
        hsa_status_string(s, &msg);
        // the copies already issued complete their own signals
        fail_job(sb, *j, SH_ERR_HIP, std::string("hsa_amd_memory_async_copy: ") + (msg ? msg : "error"), k);
        break;
      }
    }
  }
}

// Waits for `j` alone; SH_OK or its failure (recorded in the last error).
int wait_job(sh_saveback* sb, const std::shared_ptr<Job>& j) {
  {
    std::unique_lock<std::mutex> lk(sb->mu);
    sb->issued_cv.wait(lk, [&] { return j->issued; });  // a chunk job's copies are picked by the worker
  }
  bool negative = false;
  for (hsa_signal_t s : j->done) {
    hsa_signal_value_t v;
    while ((v = hsa_signal_wait_scacquire(s, HSA_SIGNAL_CONDITION_LT, 1, UINT64_MAX, HSA_WAIT_STATE_BLOCKED)) >= 1) {
    }
    negative = negative || v < 0;
  }
  std::lock_guard<std::mutex> lk(sb->mu);
  if (j->status != SH_OK) return sh::fail(j->status, "save-back ticket %llu: %s", (unsigned long long)j->id, j->error.c_str());
  if (negative) return sh::fail(SH_ERR_HIP, "save-back ticket %llu: the copy engine reported an error", (unsigned long long)j->id);
  return SH_OK;
}

bool job_done(sh_saveback* sb, const Job& j) {
  {
    std::lock_guard<std::mutex> lk(sb->mu);
    if (!j.issued) return false;
  }
  for (hsa_signal_t s : j.done)
    if (hsa_signal_load_scacquire(s) >= 1) return false;
  return true;
}

// The live jobs up to and including `ticket` (in order); SH_ERR_INVALID for a ticket never issued.
int jobs_upto(sh_saveback* sb, uint64_t ticket, std::vector<std::shared_ptr<Job>>& out, const char* who) {
  std::lock_guard<std::mutex> lk(sb->mu);
  if (ticket == 0 || ticket >= sb->next_id) return sh::fail(SH_ERR_INVALID, "%s: unknown ticket %llu", who, (unsigned long long)ticket);
  for (auto it = sb->jobs.begin(); it != sb->jobs.end() && it->first <= ticket; ++it) out.push_back(it->second);
  return SH_OK;
}

}  // namespace

extern "C" int sh_saveback_create(int device, sh_saveback** out) {
  sh::clear_error();
  if (out == nullptr) return sh::fail(SH_ERR_INVALID, "sh_saveback_create: out is NULL");
  *out = nullptr;
  SH_HIP(hipSetDevice(device));
  if (hsa_init() != HSA_STATUS_SUCCESS) return sh::fail(SH_ERR_HIP, "sh_saveback_create: hsa_init failed");
  auto sb = std::make_unique<sh_saveback>();
  sb->device = device;
  // the device's HSA agent: the owner of a small allocation made on it
  void* probe = nullptr;
  hipError_t e = hipMalloc(&probe, 256);
  if (e != hipSuccess) {
    hsa_shut_down();
    return sh::fail(SH_ERR_HIP, "sh_saveback_create: hipMalloc: %s", hipGetErrorString(e));
  }
  hsa_amd_pointer_info_t info{};
  info.size = sizeof(info);
  hsa_status_t s = hsa_amd_pointer_info(probe, &info, nullptr, nullptr, nullptr);
  (void)hipFree(probe);
  if (s != HSA_STATUS_SUCCESS || info.type == HSA_EXT_POINTER_TYPE_UNKNOWN || info.agentOwner.handle == 0) {
    hsa_shut_down();
    return sh::fail(SH_ERR_HIP, "sh_saveback_create: no HSA agent owns device %d's memory", device);
  }
  sb->gpu = info.agentOwner;
  if (hsa_agent_get_info(sb->gpu, (hsa_agent_info_t)HSA_AMD_AGENT_INFO_NEAREST_CPU, &sb->cpu) != HSA_STATUS_SUCCESS ||
      sb->cpu.handle == 0) {
    sb->cpu.handle = 0;
    hsa_iterate_agents(find_cpu, &sb->cpu);
  }
  if (sb->cpu.handle == 0) {
    hsa_shut_down();
    return sh::fail(SH_ERR_HIP, "sh_saveback_create: no CPU agent");
  }
  sh_saveback* raw = sb.release();
  raw->worker = std::thread(worker_loop, raw);
  *out = raw;
  return SH_OK;
}

extern "C" int sh_saveback_destroy(sh_saveback* sb) {
  sh::clear_error();
  if (sb == nullptr) return SH_OK;
  {
    std::lock_guard<std::mutex> lk(sb->mu);
    sb->stop = true;
  }
  sb->cv.notify_all();
  if (sb->worker.joinable()) sb->worker.join();  // issues everything still queued first
  int first = SH_OK;
  for (auto& kv : sb->jobs) {
    int st = wait_job(sb, kv.second);
    if (first == SH_OK) first = st;
  }
  sb->jobs.clear();  // the last references: each job's signal and fence go with it
  delete sb;
  hsa_shut_down();
  return first;
}

namespace {

int enqueue_job(sh_saveback* sb, const std::shared_ptr<Job>& j, void* stream, void* const* events,
                uint32_t n_events, uint64_t* ticket);

// Queues a ticket whose copies wait for an event recorded now on `stream` (events == nullptr) or
// for the caller's events.
int submit_job(sh_saveback* sb, const sh_copy_item* items, uint64_t n, void* stream, void* const* events,
               uint32_t n_events, uint64_t* ticket) {
  *ticket = 0;
  auto j = std::make_shared<Job>();
  for (uint64_t i = 0; i < n; ++i) {
    if (items[i].bytes == 0) continue;
    if (items[i].dst == nullptr || items[i].src == nullptr)
      return sh::fail(SH_ERR_INVALID, "sh_saveback_submit: item %llu has a NULL pointer", (unsigned long long)i);
    j->items.push_back(items[i]);
  }
  j->done.reserve(j->items.size());
  for (size_t k = 0; k < j->items.size(); ++k) {
    hsa_signal_t s{0};
    if (hsa_signal_create(1, 0, nullptr, &s) != HSA_STATUS_SUCCESS)
      return sh::fail(SH_ERR_HIP, "sh_saveback_submit: hsa_signal_create failed");
    j->done.push_back(s);
  }
  for (const sh_copy_item& it : j->items) j->copied += it.bytes;
  return enqueue_job(sb, j, stream, events, n_events, ticket);
}

// Gives the job its fence (an event recorded now on `stream`, or the caller's events), then
// queues it for the worker and returns its ticket.
int enqueue_job(sh_saveback* sb, const std::shared_ptr<Job>& j, void* stream, void* const* events,
                uint32_t n_events, uint64_t* ticket) {
  // A ticket without copies is complete at once (it has no signals): it gets no fence and
  // never reaches the worker, which only waits for fences and issues copies.
  const bool empty = j->items.empty() && !j->chunked;
  if (!empty && events != nullptr) {
    j->after.assign(reinterpret_cast<const hipEvent_t*>(events), reinterpret_cast<const hipEvent_t*>(events) + n_events);
  } else if (!empty) {
    hipError_t e = hipEventCreateWithFlags(&j->fence, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(j->fence, (hipStream_t)stream);
    if (e != hipSuccess) return sh::fail(SH_ERR_HIP, "sh_saveback_submit: fence event: %s", hipGetErrorString(e));
  }
  {
    std::lock_guard<std::mutex> lk(sb->mu);
    if (sb->stop) return sh::fail(SH_ERR_STATE, "sh_saveback_submit: the engine is being destroyed");
    j->id = sb->next_id++;
    sb->jobs[j->id] = j;
    if (!empty) sb->queue.push_back(j);
  }
  if (!empty) sb->cv.notify_one();
  *ticket = j->id;
  return SH_OK;
}

}  // namespace

extern "C" int sh_saveback_submit(sh_saveback* sb, const sh_copy_item* items, uint64_t n, void* stream,
                                  uint64_t* ticket) {
  sh::clear_error();
  if (sb == nullptr || ticket == nullptr || (n > 0 && items == nullptr))
    return sh::fail(SH_ERR_INVALID, "sh_saveback_submit: NULL argument");
  return submit_job(sb, items, n, stream, nullptr, 0, ticket);
}

extern "C" int sh_saveback_submit_after(sh_saveback* sb, const sh_copy_item* items, uint64_t n, void* const* events,
                                        uint32_t n_events, uint64_t* ticket) {
  sh::clear_error();
  if (sb == nullptr || ticket == nullptr || (n > 0 && items == nullptr) || (n_events > 0 && events == nullptr))
    return sh::fail(SH_ERR_INVALID, "sh_saveback_submit_after: NULL argument");
  for (uint32_t k = 0; k < n_events; ++k)
    if (events[k] == nullptr) return sh::fail(SH_ERR_INVALID, "sh_saveback_submit_after: event %u is NULL", k);
  static void* const kNone[1] = {nullptr};
  // no events: nothing to wait for (an empty, non-null list marks the caller's-events form)
  return submit_job(sb, items, n, nullptr, n_events ? events : kNone, n_events, ticket);
}

extern "C" int sh_saveback_submit_chunks(sh_saveback* sb, const sh_chunk_region* regions, uint32_t n_regions,
                                         uint32_t chunk_bytes, const uint64_t* digests, uint8_t* changed,
                                         void* digest_stream, void* const* events, uint32_t n_events, void* stream,
                                         uint64_t* ticket) {
  static const char* who = "sh_saveback_submit_chunks";
  sh::clear_error();
  if (sb == nullptr || ticket == nullptr || (n_regions > 0 && regions == nullptr) || (n_events > 0 && events == nullptr))
    return sh::fail(SH_ERR_INVALID, "%s: NULL argument", who);
  *ticket = 0;
  if (chunk_bytes == 0 || chunk_bytes % 16 != 0)
    return sh::fail(SH_ERR_INVALID, "%s: chunk_bytes %u is not a positive multiple of 16", who, chunk_bytes);
  if (digests != nullptr && changed == nullptr) return sh::fail(SH_ERR_INVALID, "%s: digests without `changed`", who);
  auto j = std::make_shared<Job>();
  for (uint32_t i = 0; i < n_regions; ++i) {
    const sh_chunk_region& r = regions[i];
    if (r.bytes == 0) continue;
    if (r.host_dst == nullptr || r.dev_src == nullptr)
      return sh::fail(SH_ERR_INVALID, "%s: region %u has a NULL buffer", who, i);
    const uint64_t n = r.bytes / chunk_bytes + (r.bytes % chunk_bytes != 0 ? 1 : 0);
    if (n > sh::kMaxDigestChunks || r.first_chunk > UINT64_MAX / 16 - n)
      return sh::fail(SH_ERR_INVALID, "%s: region %u has too many chunks of %u bytes", who, i, chunk_bytes);
    j->regions.push_back(r);
  }
  for (uint32_t k = 0; k < n_events; ++k)
    if (events[k] == nullptr) return sh::fail(SH_ERR_INVALID, "%s: event %u is NULL", who, k);
  if (j->regions.empty()) return enqueue_job(sb, j, stream, n_events ? events : nullptr, n_events, ticket);
  j->chunked = true;
  j->issued = false;
  j->chunk = chunk_bytes;
  j->digests = digests;
  j->changed = changed;
  if (digests == nullptr) return enqueue_job(sb, j, stream, n_events ? events : nullptr, n_events, ticket);
  // The comparison goes on digest_stream now, after the caller's events (or after the work
  // queued on `stream`), and the job's fence after it: it is not queued behind work that
  // digest_stream receives later, and the worker only reads the flags.
  hipStream_t ds = (hipStream_t)digest_stream;
  hipError_t e = hipSuccess;
  if (n_events > 0) {
    for (uint32_t k = 0; k < n_events && e == hipSuccess; ++k) e = hipStreamWaitEvent(ds, (hipEvent_t)events[k], 0);
  } else if ((hipStream_t)stream != ds) {
    e = hipEventCreateWithFlags(&j->order, hipEventDisableTiming);  // lives with the job
    if (e == hipSuccess) e = hipEventRecord(j->order, (hipStream_t)stream);
    if (e == hipSuccess) e = hipStreamWaitEvent(ds, j->order, 0);
  }
  if (e != hipSuccess) return sh::fail(SH_ERR_HIP, "%s: ordering the comparison: %s", who, hipGetErrorString(e));
  for (const sh_chunk_region& r : j->regions) {
    int st = sh::launch_block_changed(r.dev_src, r.bytes, chunk_bytes, digests + 2 * r.first_chunk,
                                      changed + r.first_chunk, ds);
    if (st != SH_OK) return st;
  }
  return enqueue_job(sb, j, digest_stream, nullptr, 0, ticket);
}

extern "C" int sh_saveback_ticket_bytes(sh_saveback* sb, uint64_t ticket, uint64_t* bytes) {
  sh::clear_error();
  if (sb == nullptr || bytes == nullptr) return sh::fail(SH_ERR_INVALID, "sh_saveback_ticket_bytes: NULL argument");
  std::shared_ptr<Job> j;
  {
    std::lock_guard<std::mutex> lk(sb->mu);
    auto it = sb->jobs.find(ticket);
    if (it == sb->jobs.end()) return sh::fail(SH_ERR_INVALID, "sh_saveback_ticket_bytes: unknown or released ticket");
    j = it->second;
  }
  int st = wait_job(sb, j);
  if (st != SH_OK) return st;
  std::lock_guard<std::mutex> lk(sb->mu);
  *bytes = j->copied;
  return SH_OK;
}

extern "C" int sh_saveback_query(sh_saveback* sb, uint64_t ticket) {
  sh::clear_error();
  if (sb == nullptr) return sh::fail(SH_ERR_INVALID, "sh_saveback_query: NULL engine");
  std::vector<std::shared_ptr<Job>> js;
  int st = jobs_upto(sb, ticket, js, "sh_saveback_query");
  if (st != SH_OK) return st;
  for (const auto& j : js) {
    if (!job_done(sb, *j)) return SH_ERR_NOT_READY;
    st = wait_job(sb, j);  // every signal at its final value: returns at once
    if (st != SH_OK) return st;
  }
  return SH_OK;
}

extern "C" int sh_saveback_wait(sh_saveback* sb, uint64_t ticket) {
  sh::clear_error();
  if (sb == nullptr) return sh::fail(SH_ERR_INVALID, "sh_saveback_wait: NULL engine");
  std::vector<std::shared_ptr<Job>> js;
  int st = jobs_upto(sb, ticket, js, "sh_saveback_wait");
  if (st != SH_OK) return st;
  for (const auto& j : js) {
    st = wait_job(sb, j);
    if (st != SH_OK) return st;
  }
  return SH_OK;
}

extern "C" int sh_saveback_release(sh_saveback* sb, uint64_t ticket) {
  sh::clear_error();
  if (sb == nullptr) return sh::fail(SH_ERR_INVALID, "sh_saveback_release: NULL engine");
  std::shared_ptr<Job> j;
  {
    std::lock_guard<std::mutex> lk(sb->mu);
    auto it = sb->jobs.find(ticket);
    if (it == sb->jobs.end()) {
      if (ticket == 0 || ticket >= sb->next_id)
        return sh::fail(SH_ERR_INVALID, "sh_saveback_release: unknown ticket %llu", (unsigned long long)ticket);
      return SH_OK;  // released before
    }
    j = it->second;
  }
  // Waits for its own copies only (they read and write the caller's buffers), then drops the
  // map's reference. The signal and fence live on while the worker or a waiter holds the job.
  int st = wait_job(sb, j);
  {
    std::lock_guard<std::mutex> lk(sb->mu);
    sb->jobs.erase(ticket);
  }
  return st;
}

namespace {
uint64_t ticks_to_ns(uint64_t ticks) {
  static uint64_t freq = 0;
  if (freq == 0 && hsa_system_get_info(HSA_SYSTEM_INFO_TIMESTAMP_FREQUENCY, &freq) != HSA_STATUS_SUCCESS) freq = 0;
  if (freq == 0) return 0;
  return (uint64_t)((__uint128_t)ticks * 1000000000ull / freq);
}
}  // namespace

extern "C" int sh_saveback_set_timing(sh_saveback* sb, int enable) {
  sh::clear_error();
  if (sb == nullptr) return sh::fail(SH_ERR_INVALID, "sh_saveback_set_timing: NULL engine");
  // the runtime-wide switch stays on once set: the HIP runtime's own copies may rely on it
  if (enable && hsa_amd_profiling_async_copy_enable(true) != HSA_STATUS_SUCCESS)
    return sh::fail(SH_ERR_HIP, "sh_saveback_set_timing: hsa_amd_profiling_async_copy_enable failed");
  sb->timing.store(enable != 0);
  return SH_OK;
}

extern "C" int sh_saveback_clock_ns(uint64_t* ns) {
  sh::clear_error();
  if (ns == nullptr) return sh::fail(SH_ERR_INVALID, "sh_saveback_clock_ns: NULL argument");
  uint64_t t = 0;
  if (hsa_system_get_info(HSA_SYSTEM_INFO_TIMESTAMP, &t) != HSA_STATUS_SUCCESS)
    return sh::fail(SH_ERR_HIP, "sh_saveback_clock_ns: hsa_system_get_info failed");
  *ns = ticks_to_ns(t);
  return SH_OK;
}

extern "C" int sh_saveback_ticket_times(sh_saveback* sb, uint64_t ticket, uint64_t* out2) {
  sh::clear_error();
  if (sb == nullptr || out2 == nullptr) return sh::fail(SH_ERR_INVALID, "sh_saveback_ticket_times: NULL argument");
  std::shared_ptr<Job> j;
  {
    std::lock_guard<std::mutex> lk(sb->mu);
    auto it = sb->jobs.find(ticket);
    if (it == sb->jobs.end()) return sh::fail(SH_ERR_INVALID, "sh_saveback_ticket_times: unknown or released ticket");
    j = it->second;
  }
  int st = wait_job(sb, j);
  if (st != SH_OK) return st;
  out2[0] = out2[1] = 0;
  if (j->items.empty()) return SH_OK;
  // each copy's signal holds that copy's engine start and end times
  uint64_t start = UINT64_MAX, end = 0;
  for (hsa_signal_t s : j->done) {
    hsa_amd_profiling_async_copy_time_t t{};
    if (hsa_amd_profiling_get_async_copy_time(s, &t) != HSA_STATUS_SUCCESS || t.end == 0)
      return sh::fail(SH_ERR_STATE, "sh_saveback_ticket_times: no copy times (the ticket was submitted without "
                                    "timing, or a tool replaced its copies' completion signals)");
    start = std::min<uint64_t>(start, t.start);
    end = std::max<uint64_t>(end, t.end);
  }
  out2[0] = ticks_to_ns(start);
  out2[1] = ticks_to_ns(end);
  return SH_OK;
}
