// A CPU stand-in for the HIP and HSA runtime calls the library's host code makes, for the
// sanitizer builds in this directory (never part of the library). It lets the threaded engines
// (block loader, save-back engine, turbo engine, VMM allocator) run under the thread and address
// sanitizers on a machine without a GPU, with the same ordering rules as the real runtime:
//
// - device memory is host memory; hipMalloc / hipHostMalloc allocate it, hipFree / hipHostFree
//   first wait for every stream (as HIP's implicit device synchronisation does);
// - a stream is a worker thread running its queue in order: copies, kernel launches, event
//   records and waits on other streams' events all run there, so anything the library reads
//   before waiting for the work that writes it is a data race the thread sanitizer reports;
// - an event completes when its stream's worker reaches the record; host waits (synchronize,
//   query) and device waits (hipStreamWaitEvent) follow it;
// - the HSA SDMA copy (hsa_amd_memory_async_copy) runs on an engine thread of its own, waits
//   for its dependency signals and decrements its completion signal;
// - the module API resolves every kernel by name; the digest kernels run the library's own host
//   digest (sh_block_digest_host) on the stream, every other kernel does nothing;
// - VMM reservations are PROT_NONE mappings, hipMemMap maps fresh zero pages into them and
//   hipMemUnmap takes the pages away again, so a read of an evicted region faults.
//
// fake_hip_fail_next(name, n) makes the next n calls of one entry point fail, for the tests of
// the engines' error paths; fake_hip_sdma_delay_us(us) makes every SDMA copy take that much longer.

#include <hip/hip_runtime.h>
#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>
#include <sys/mman.h>

#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <string>
#include <thread>
#include <vector>

#include "stagehand_native.h"

namespace {

uint64_t now_ns() {
  return (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
             std::chrono::steady_clock::now().time_since_epoch())
      .count();
}

// ── failure injection ─────────────────────────────────────────────────────

std::mutex g_fail_mu;
std::map<std::string, int>* g_fail = nullptr;

bool should_fail(const char* name) {
  std::lock_guard<std::mutex> lk(g_fail_mu);
  if (g_fail == nullptr) return false;
  auto it = g_fail->find(name);
  if (it == g_fail->end() || it->second <= 0) return false;
  --it->second;
  return true;
}

// ── events ────────────────────────────────────────────────────────────────

struct EventState {
  std::mutex mu;
  std::condition_variable cv;
  uint64_t recorded = 0;   // records issued
  uint64_t completed = 0;  // records the stream has reached
  uint64_t time_ns = 0;    // when the latest record completed
};

struct FakeEvent {
  std::shared_ptr<EventState> st = std::make_shared<EventState>();
};

// ── streams ───────────────────────────────────────────────────────────────

struct FakeStream {
  std::mutex mu;
  std::condition_variable cv, idle_cv;
  std::deque<std::function<void()>> q;
  bool stop = false;
  bool busy = false;
  std::thread worker;

  FakeStream() { worker = std::thread([this] { run(); }); }
  ~FakeStream() {
    {
      std::lock_guard<std::mutex> lk(mu);
      stop = true;
    }
    cv.notify_all();
    worker.join();
  }
  void push(std::function<void()> fn) {
    {
      std::lock_guard<std::mutex> lk(mu);
      q.push_back(std::move(fn));
    }
    cv.notify_all();
  }
  void drain() {
    std::unique_lock<std::mutex> lk(mu);
    idle_cv.wait(lk, [&] { return q.empty() && !busy; });
  }
  void run() {
    for (;;) {
      std::function<void()> fn;
      {
        std::unique_lock<std::mutex> lk(mu);
        cv.wait(lk, [&] { return stop || !q.empty(); });
        if (q.empty()) return;  // stop, and nothing left to run
        fn = std::move(q.front());
        q.pop_front();
        busy = true;
      }
      fn();
      {
        std::lock_guard<std::mutex> lk(mu);
        busy = false;
      }
      idle_cv.notify_all();
    }
  }
};

std::mutex g_streams_mu;
// every live stream, the null stream included; the map owns them, and drain_all holds a reference
// to each stream it drains, so a stream destroyed meanwhile is deleted once that drain ends
std::map<FakeStream*, std::shared_ptr<FakeStream>>* g_streams = nullptr;
FakeStream* g_null = nullptr;

FakeStream* stream_of(hipStream_t s) {
  if (s != nullptr) return reinterpret_cast<FakeStream*>(s);
  std::lock_guard<std::mutex> lk(g_streams_mu);
  if (g_null == nullptr) {
    auto sp = std::make_shared<FakeStream>();
    g_null = sp.get();
    if (g_streams == nullptr) g_streams = new std::map<FakeStream*, std::shared_ptr<FakeStream>>();
    (*g_streams)[g_null] = std::move(sp);
  }
  return g_null;
}

void drain_all() {
  std::vector<std::shared_ptr<FakeStream>> all;
  {
    std::lock_guard<std::mutex> lk(g_streams_mu);
    if (g_streams != nullptr)
      for (const auto& kv : *g_streams) all.push_back(kv.second);
  }
  for (const auto& s : all) s->drain();
}

void complete(const std::shared_ptr<EventState>& st, uint64_t gen) {
  {
    std::lock_guard<std::mutex> lk(st->mu);
    if (gen > st->completed) st->completed = gen;
    st->time_ns = now_ns();
  }
  st->cv.notify_all();
}

void wait_for(const std::shared_ptr<EventState>& st, uint64_t gen) {
  std::unique_lock<std::mutex> lk(st->mu);
  st->cv.wait(lk, [&] { return st->completed >= gen; });
}

// ── modules ───────────────────────────────────────────────────────────────

struct FakeFunction {
  std::string name;
};
struct FakeModule {
  std::vector<uint8_t> scratch = std::vector<uint8_t>(SH_UNPACK_NOALLOC_SCRATCH_BYTES);
  std::vector<std::unique_ptr<FakeFunction>> functions;  // freed with the module
};

// ── HSA signals and the SDMA engine ───────────────────────────────────────

struct FakeSignal {
  std::mutex mu;
  std::condition_variable cv;
  hsa_signal_value_t value;
  uint64_t start = 0, end = 0;  // copy times (ns)
};

FakeSignal* sig(hsa_signal_t s) { return reinterpret_cast<FakeSignal*>(s.handle); }

std::mutex g_sdma_mu;
FakeStream* g_sdma = nullptr;
FakeStream* sdma() {
  std::lock_guard<std::mutex> lk(g_sdma_mu);
  if (g_sdma == nullptr) g_sdma = new FakeStream();  // never destroyed, like the engines of a GPU
  return g_sdma;
}

std::atomic<int> g_hsa_refs{0};
std::atomic<unsigned> g_sdma_delay_us{0};  // a slower copy engine (fake_hip_sdma_delay_us)

constexpr uint64_t kGpuAgent = 1, kCpuAgent = 2;

// ── VMM ───────────────────────────────────────────────────────────────────

struct FakeAlloc {
  size_t size;
};
std::atomic<uint64_t> g_allocated{0};

}  // namespace

extern "C" {

void fake_hip_sdma_delay_us(unsigned us) { g_sdma_delay_us.store(us); }

int fake_hip_fail_pending(const char* name) {
  std::lock_guard<std::mutex> lk(g_fail_mu);
  if (g_fail == nullptr) return 0;
  auto it = g_fail->find(name);
  return it == g_fail->end() ? 0 : it->second;
}

void fake_hip_fail_next(const char* name, int n) {
  std::lock_guard<std::mutex> lk(g_fail_mu);
  if (g_fail == nullptr) g_fail = new std::map<std::string, int>();
  (*g_fail)[name] = n;
}

// ── device, errors ────────────────────────────────────────────────────────

const char* hipGetErrorString(hipError_t e) {
  static thread_local char buf[64];
  std::snprintf(buf, sizeof buf, "fake HIP error %d", (int)e);
  return buf;
}

hipError_t hipGetDevice(int* d) {
  if (d == nullptr) return hipErrorInvalidValue;
  *d = 0;
  return hipSuccess;
}
hipError_t hipSetDevice(int d) { return d == 0 ? hipSuccess : hipErrorInvalidDevice; }
hipError_t hipGetDeviceCount(int* n) {
  *n = 1;
  return hipSuccess;
}
hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t attr, int dev) {
  if (dev != 0) return hipErrorInvalidDevice;
  *v = attr == hipDeviceAttributeVirtualMemoryManagementSupported ? 1 : 0;
  return hipSuccess;
}
hipError_t hipMemGetInfo(size_t* free_b, size_t* total) {
  *total = (size_t)288 << 30;
  *free_b = *total - (size_t)g_allocated.load();
  return hipSuccess;
}
hipError_t hipDeviceSynchronize(void) {
  drain_all();
  return hipSuccess;
}

// ── memory ────────────────────────────────────────────────────────────────

hipError_t hipMalloc(void** p, size_t n) {
  if (should_fail("hipMalloc")) return hipErrorOutOfMemory;
  *p = std::aligned_alloc(256, (n + 255) / 256 * 256 + 256);
  return *p ? hipSuccess : hipErrorOutOfMemory;
}
hipError_t hipFree(void* p) {
  drain_all();
  std::free(p);
  return hipSuccess;
}
hipError_t hipHostMalloc(void** p, size_t n, unsigned int) {
  if (should_fail("hipHostMalloc")) return hipErrorOutOfMemory;
  *p = std::aligned_alloc(4096, (n + 4095) / 4096 * 4096 + 4096);
  return *p ? hipSuccess : hipErrorOutOfMemory;
}
hipError_t hipHostFree(void* p) {
  drain_all();
  std::free(p);
  return hipSuccess;
}
hipError_t hipMemcpy(void* dst, const void* src, size_t n, hipMemcpyKind) {
  drain_all();
  std::memcpy(dst, src, n);
  return hipSuccess;
}
hipError_t hipMemcpyAsync(void* dst, const void* src, size_t n, hipMemcpyKind, hipStream_t s) {
  if (should_fail("hipMemcpyAsync")) return hipErrorInvalidValue;
  stream_of(s)->push([=] { std::memcpy(dst, src, n); });
  return hipSuccess;
}

// ── streams and events ────────────────────────────────────────────────────

hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned int) {
  auto sp = std::make_shared<FakeStream>();
  FakeStream* fs = sp.get();
  {
    std::lock_guard<std::mutex> lk(g_streams_mu);
    if (g_streams == nullptr) g_streams = new std::map<FakeStream*, std::shared_ptr<FakeStream>>();
    (*g_streams)[fs] = std::move(sp);
  }
  *s = reinterpret_cast<hipStream_t>(fs);
  return hipSuccess;
}
hipError_t hipStreamDestroy(hipStream_t s) {
  if (s == nullptr) return hipErrorInvalidHandle;
  FakeStream* fs = reinterpret_cast<FakeStream*>(s);
  std::shared_ptr<FakeStream> sp;
  {
    std::lock_guard<std::mutex> lk(g_streams_mu);
    auto it = g_streams->find(fs);
    if (it == g_streams->end()) return hipErrorInvalidHandle;
    sp = std::move(it->second);
    g_streams->erase(it);
  }
  sp.reset();  // the last reference runs what is queued, then joins
  return hipSuccess;
}
hipError_t hipStreamSynchronize(hipStream_t s) {
  stream_of(s)->drain();
  return hipSuccess;
}
hipError_t hipStreamIsCapturing(hipStream_t, hipStreamCaptureStatus* st) {
  *st = hipStreamCaptureStatusNone;
  return hipSuccess;
}
hipError_t hipEventCreateWithFlags(hipEvent_t* e, unsigned) {
  *e = reinterpret_cast<hipEvent_t>(new FakeEvent());
  return hipSuccess;
}
hipError_t hipEventCreate(hipEvent_t* e) { return hipEventCreateWithFlags(e, 0); }
hipError_t hipEventDestroy(hipEvent_t e) {
  delete reinterpret_cast<FakeEvent*>(e);  // queued records keep the state alive
  return hipSuccess;
}
hipError_t hipEventRecord(hipEvent_t e, hipStream_t s) {
  if (should_fail("hipEventRecord")) return hipErrorInvalidValue;
  std::shared_ptr<EventState> st = reinterpret_cast<FakeEvent*>(e)->st;
  uint64_t gen;
  {
    std::lock_guard<std::mutex> lk(st->mu);
    gen = ++st->recorded;
  }
  stream_of(s)->push([st, gen] { complete(st, gen); });
  return hipSuccess;
}
hipError_t hipEventSynchronize(hipEvent_t e) {
  std::shared_ptr<EventState> st = reinterpret_cast<FakeEvent*>(e)->st;
  uint64_t gen;
  {
    std::lock_guard<std::mutex> lk(st->mu);
    gen = st->recorded;
  }
  wait_for(st, gen);
  return hipSuccess;
}
hipError_t hipEventQuery(hipEvent_t e) {
  std::shared_ptr<EventState> st = reinterpret_cast<FakeEvent*>(e)->st;
  std::lock_guard<std::mutex> lk(st->mu);
  return st->completed >= st->recorded ? hipSuccess : hipErrorNotReady;
}
hipError_t hipEventElapsedTime(float* ms, hipEvent_t a, hipEvent_t b) {
  std::shared_ptr<EventState> sa = reinterpret_cast<FakeEvent*>(a)->st, sb = reinterpret_cast<FakeEvent*>(b)->st;
  std::scoped_lock lk(sa->mu, sb->mu);
  if (sa->completed < sa->recorded || sb->completed < sb->recorded) return hipErrorNotReady;
  *ms = (float)((double)((int64_t)sb->time_ns - (int64_t)sa->time_ns) * 1e-6);
  return hipSuccess;
}
hipError_t hipStreamWaitEvent(hipStream_t s, hipEvent_t e, unsigned int) {
  std::shared_ptr<EventState> st = reinterpret_cast<FakeEvent*>(e)->st;
  uint64_t gen;
  {
    std::lock_guard<std::mutex> lk(st->mu);
    gen = st->recorded;
  }
  if (gen == 0) return hipSuccess;
  stream_of(s)->push([st, gen] { wait_for(st, gen); });
  return hipSuccess;
}

// ── modules ───────────────────────────────────────────────────────────────

hipError_t hipModuleLoadData(hipModule_t* m, const void* image) {
  if (image == nullptr) return hipErrorInvalidImage;
  *m = reinterpret_cast<hipModule_t>(new FakeModule());
  return hipSuccess;
}
hipError_t hipModuleUnload(hipModule_t m) {
  drain_all();
  delete reinterpret_cast<FakeModule*>(m);
  return hipSuccess;
}
hipError_t hipModuleGetFunction(hipFunction_t* f, hipModule_t m, const char* name) {
  FakeModule* fm = reinterpret_cast<FakeModule*>(m);
  fm->functions.push_back(std::make_unique<FakeFunction>(FakeFunction{name}));
  *f = reinterpret_cast<hipFunction_t>(fm->functions.back().get());
  return hipSuccess;
}
hipError_t hipModuleGetGlobal(hipDeviceptr_t* p, size_t* bytes, hipModule_t m, const char* name) {
  if (std::strcmp(name, "scratch") != 0) return hipErrorNotFound;
  FakeModule* fm = reinterpret_cast<FakeModule*>(m);
  *p = fm->scratch.data();
  *bytes = fm->scratch.size();
  return hipSuccess;
}
hipError_t hipModuleLaunchKernel(hipFunction_t f, unsigned int gx, unsigned int, unsigned int, unsigned int,
                                 unsigned int, unsigned int, unsigned int, hipStream_t s, void** params, void**) {
  if (should_fail("hipModuleLaunchKernel")) return hipErrorLaunchFailure;
  const std::string& name = reinterpret_cast<FakeFunction*>(f)->name;
  if (gx == 0) return hipErrorInvalidConfiguration;
  if (name == "sh_digest_kernel") {
    const uint8_t* buf = *(const uint8_t**)params[0];
    const uint64_t bytes = *(const uint64_t*)params[1];
    const uint64_t chunk = *(const uint64_t*)params[2];
    uint64_t* digests = *(uint64_t**)params[3];
    stream_of(s)->push([=] { (void)sh_block_digest_host(buf, bytes, (uint32_t)chunk, digests); });
  } else if (name == "sh_digest_compare_kernel") {
    const uint8_t* buf = *(const uint8_t**)params[0];
    const uint64_t bytes = *(const uint64_t*)params[1];
    const uint64_t chunk = *(const uint64_t*)params[2];
    const uint64_t* digests = *(const uint64_t**)params[3];
    uint8_t* changed = *(uint8_t**)params[4];
    stream_of(s)->push([=] {
      const uint64_t n = (bytes + chunk - 1) / chunk;
      std::vector<uint64_t> now(2 * n);
      (void)sh_block_digest_host(buf, bytes, (uint32_t)chunk, now.data());
      for (uint64_t c = 0; c < n; ++c)
        changed[c] = (now[2 * c] != digests[2 * c] || now[2 * c + 1] != digests[2 * c + 1]) ? 1 : 0;
    });
  } else {
    stream_of(s)->push([] {});  // the unpack kernels: no CPU form here
  }
  return hipSuccess;
}

// ── VMM ───────────────────────────────────────────────────────────────────

hipError_t hipMemGetAllocationGranularity(size_t* g, const hipMemAllocationProp*, hipMemAllocationGranularity_flags) {
  *g = 4096;
  return hipSuccess;
}
hipError_t hipMemAddressReserve(void** p, size_t size, size_t, void*, unsigned long long) {
  void* r = mmap(nullptr, size, PROT_NONE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
  if (r == MAP_FAILED) return hipErrorOutOfMemory;
  *p = r;
  return hipSuccess;
}
hipError_t hipMemAddressFree(void* p, size_t size) { return munmap(p, size) == 0 ? hipSuccess : hipErrorInvalidValue; }
hipError_t hipMemCreate(hipMemGenericAllocationHandle_t* h, size_t size, const hipMemAllocationProp*,
                        unsigned long long) {
  if (should_fail("hipMemCreate")) return hipErrorOutOfMemory;
  *h = reinterpret_cast<hipMemGenericAllocationHandle_t>(new FakeAlloc{size});
  g_allocated.fetch_add(size);
  return hipSuccess;
}
hipError_t hipMemRelease(hipMemGenericAllocationHandle_t h) {
  FakeAlloc* a = reinterpret_cast<FakeAlloc*>(h);
  g_allocated.fetch_sub(a->size);
  delete a;
  return hipSuccess;
}
hipError_t hipMemMap(void* p, size_t size, size_t, hipMemGenericAllocationHandle_t, unsigned long long) {
  void* r = mmap(p, size, PROT_READ | PROT_WRITE, MAP_FIXED | MAP_PRIVATE | MAP_ANONYMOUS, -1, 0);
  return r == p ? hipSuccess : hipErrorOutOfMemory;
}
hipError_t hipMemSetAccess(void*, size_t, const hipMemAccessDesc*, size_t) { return hipSuccess; }
hipError_t hipMemUnmap(void* p, size_t size) {
  drain_all();  // no queued copy may still write the region
  void* r = mmap(p, size, PROT_NONE, MAP_FIXED | MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
  return r == p ? hipSuccess : hipErrorInvalidValue;
}

// ── HSA ───────────────────────────────────────────────────────────────────

hsa_status_t hsa_init(void) {
  g_hsa_refs.fetch_add(1);
  return HSA_STATUS_SUCCESS;
}
hsa_status_t hsa_shut_down(void) {
  return g_hsa_refs.fetch_sub(1) > 0 ? HSA_STATUS_SUCCESS : HSA_STATUS_ERROR_NOT_INITIALIZED;
}
hsa_status_t hsa_status_string(hsa_status_t, const char** s) {
  *s = "fake HSA error";
  return HSA_STATUS_SUCCESS;
}
hsa_status_t hsa_system_get_info(hsa_system_info_t attr, void* value) {
  if (attr == HSA_SYSTEM_INFO_TIMESTAMP) {
    *(uint64_t*)value = now_ns();
    return HSA_STATUS_SUCCESS;
  }
  if (attr == HSA_SYSTEM_INFO_TIMESTAMP_FREQUENCY) {
    *(uint64_t*)value = 1000000000ull;
    return HSA_STATUS_SUCCESS;
  }
  return HSA_STATUS_ERROR_INVALID_ARGUMENT;
}
hsa_status_t hsa_amd_pointer_info(const void* ptr, hsa_amd_pointer_info_t* info, void* (*)(size_t), uint32_t*,
                                  hsa_agent_t**) {
  if (ptr == nullptr || info == nullptr) return HSA_STATUS_ERROR_INVALID_ARGUMENT;
  info->type = HSA_EXT_POINTER_TYPE_HSA;
  info->agentOwner.handle = kGpuAgent;
  return HSA_STATUS_SUCCESS;
}
hsa_status_t hsa_agent_get_info(hsa_agent_t agent, hsa_agent_info_t attr, void* value) {
  if (attr == HSA_AGENT_INFO_DEVICE) {
    *(hsa_device_type_t*)value = agent.handle == kCpuAgent ? HSA_DEVICE_TYPE_CPU : HSA_DEVICE_TYPE_GPU;
    return HSA_STATUS_SUCCESS;
  }
  if ((int)attr == (int)HSA_AMD_AGENT_INFO_NEAREST_CPU && agent.handle == kGpuAgent) {
    ((hsa_agent_t*)value)->handle = kCpuAgent;
    return HSA_STATUS_SUCCESS;
  }
  return HSA_STATUS_ERROR_INVALID_ARGUMENT;
}
hsa_status_t hsa_iterate_agents(hsa_status_t (*cb)(hsa_agent_t, void*), void* data) {
  for (uint64_t a : {kGpuAgent, kCpuAgent}) {
    const hsa_status_t st = cb(hsa_agent_t{a}, data);
    if (st == HSA_STATUS_INFO_BREAK) return HSA_STATUS_SUCCESS;
    if (st != HSA_STATUS_SUCCESS) return st;
  }
  return HSA_STATUS_SUCCESS;
}
hsa_status_t hsa_signal_create(hsa_signal_value_t v, uint32_t, const hsa_agent_t*, hsa_signal_t* s) {
  if (should_fail("hsa_signal_create")) return HSA_STATUS_ERROR_OUT_OF_RESOURCES;
  FakeSignal* f = new FakeSignal();
  f->value = v;
  s->handle = reinterpret_cast<uint64_t>(f);
  return HSA_STATUS_SUCCESS;
}
hsa_status_t hsa_signal_destroy(hsa_signal_t s) {
  delete sig(s);
  return HSA_STATUS_SUCCESS;
}
hsa_signal_value_t hsa_signal_load_scacquire(hsa_signal_t s) {
  FakeSignal* f = sig(s);
  std::lock_guard<std::mutex> lk(f->mu);
  return f->value;
}
void hsa_signal_subtract_screlease(hsa_signal_t s, hsa_signal_value_t v) {
  FakeSignal* f = sig(s);
  // Notified under the lock: a waiter that sees the new value may destroy the signal at once, so
  // nothing here may touch it after the lock is released.
  std::lock_guard<std::mutex> lk(f->mu);
  f->value -= v;
  f->cv.notify_all();
}
hsa_signal_value_t hsa_signal_wait_scacquire(hsa_signal_t s, hsa_signal_condition_t cond, hsa_signal_value_t cmp,
                                             uint64_t, hsa_wait_state_t) {
  FakeSignal* f = sig(s);
  auto holds = [&] {
    switch (cond) {
      case HSA_SIGNAL_CONDITION_EQ: return f->value == cmp;
      case HSA_SIGNAL_CONDITION_NE: return f->value != cmp;
      case HSA_SIGNAL_CONDITION_LT: return f->value < cmp;
      case HSA_SIGNAL_CONDITION_GTE: return f->value >= cmp;
    }
    return true;
  };
  std::unique_lock<std::mutex> lk(f->mu);
  f->cv.wait(lk, holds);
  return f->value;
}
hsa_status_t hsa_amd_memory_async_copy(void* dst, hsa_agent_t, const void* src, hsa_agent_t, size_t size,
                                       uint32_t n_deps, const hsa_signal_t* deps, hsa_signal_t done) {
  if (should_fail("hsa_amd_memory_async_copy")) return HSA_STATUS_ERROR_OUT_OF_RESOURCES;
  std::vector<hsa_signal_t> d(deps, deps + n_deps);
  sdma()->push([=] {
    for (hsa_signal_t s : d) (void)hsa_signal_wait_scacquire(s, HSA_SIGNAL_CONDITION_LT, 1, UINT64_MAX,
                                                              HSA_WAIT_STATE_BLOCKED);
    FakeSignal* f = sig(done);
    if (const unsigned us = g_sdma_delay_us.load()) std::this_thread::sleep_for(std::chrono::microseconds(us));
    const uint64_t t0 = now_ns();
    std::memcpy(dst, src, size);
    {
      std::lock_guard<std::mutex> lk(f->mu);
      f->start = t0;
      f->end = now_ns();
    }
    hsa_signal_subtract_screlease(done, 1);
  });
  return HSA_STATUS_SUCCESS;
}
hsa_status_t hsa_amd_profiling_async_copy_enable(bool) { return HSA_STATUS_SUCCESS; }
hsa_status_t hsa_amd_profiling_get_async_copy_time(hsa_signal_t s, hsa_amd_profiling_async_copy_time_t* t) {
  FakeSignal* f = sig(s);
  std::lock_guard<std::mutex> lk(f->mu);
  t->start = f->start;
  t->end = f->end;
  return HSA_STATUS_SUCCESS;
}

}  // extern "C"
