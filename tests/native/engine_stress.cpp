// Multi-threaded stress of the library's threaded engines, built with the thread and with the
// address + undefined-behaviour sanitizers against the CPU stand-in runtime (fake_hip.cpp; the
// Makefile in this directory builds it, tests/test_sanitizers.py runs it).
//
// - Block loader: two loaders on one pinned pool, each driven by its own thread, with up to
//   four tickets in flight and finished in varying orders (query, device wait, host sync):
//   zero-byte tickets, host pieces, file ranges, pinned pieces written by a save-back ticket
//   that the loader's worker waits for, and loads with chunk digests.
// - Save-back engine: one thread submits (plain, after events, changed chunks with digests,
//   zero items) while another waits for and releases the tickets, later ones before earlier
//   ones; destroy with tickets still queued.
// - Turbo engine: forward and backward passes with every block changed on the device after its
//   step and written back on the SDMA engine in changed chunks, with the copy engine slowed so
//   that look-ahead copies are deferred; a failed copy (injected) must leave the block back on
//   the host with its slot free, and the engine must go on working.
// - VMM allocator: three threads take and release handles on eight regions under a ceiling of
//   four while a fourth prefetches, changes priorities and reads statistics.
// Every byte that moves is checked; the sanitizers fail the run on a race, a use after free,
// an out-of-bounds access or undefined behaviour.
//
// Reference protocols exercised: vmm_src/allocator.rs:227-273 (claim and refcount re-check),
// vmm_src/eviction.rs:50-78 (CAS eviction), vmm_src/prefetch.rs:22-46 (prefetch worker),
// turbo_src/engine.rs:202-341 (window, write-back, slot reuse).

#include <hip/hip_runtime.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "stagehand_native.h"

extern "C" void fake_hip_fail_next(const char* name, int n);
extern "C" void fake_hip_sdma_delay_us(unsigned us);
extern "C" int fake_hip_fail_pending(const char* name);

namespace {

std::atomic<int> g_failures{0};

void check(bool ok, const char* what, long detail = -1) {
  if (!ok) {
    std::fprintf(stderr, "FAIL: %s [%ld] (last error: %s)\n", what, detail, sh_last_error());
    g_failures.fetch_add(1);
  }
}

struct Rng {
  uint64_t s;
  explicit Rng(uint64_t seed) : s(seed * 0x9E3779B97F4A7C15ull + 1) {}
  uint64_t next() {
    s ^= s << 13;
    s ^= s >> 7;
    s ^= s << 17;
    return s;
  }
  uint64_t below(uint64_t n) { return n ? next() % n : 0; }
};

void* dmalloc(size_t n) {
  void* p = nullptr;
  check(hipMalloc(&p, n ? n : 1) == hipSuccess, "hipMalloc");
  return p;
}
void* hmalloc(size_t n) {
  void* p = nullptr;
  check(hipHostMalloc(&p, n ? n : 1, 0) == hipSuccess, "hipHostMalloc");
  return p;
}
void fill(std::vector<uint8_t>& v, Rng& r) {
  for (size_t i = 0; i < v.size(); ++i) v[i] = (uint8_t)(r.next() >> 24);
}

// ── block loader ──────────────────────────────────────────────────────────

struct Load {
  uint64_t ticket = 0;
  int kind = 0;
  std::vector<uint8_t> src, want;
  void* dst = nullptr;
  uint64_t bytes = 0;
  void* pinned = nullptr;
  void* dev_src = nullptr;
  uint64_t sb_ticket = 0;
  uint64_t* digest = nullptr;
  uint32_t chunk = 4096;
};

void finish_load(sh_loader* L, sh_saveback* sb, hipStream_t s, Load& ld, Rng& r) {
  // a load's unpack and digests are queued by whichever of these comes first; a release with no
  // wait before it still leaves the destination and the digests written
  bool released = false;
  // the copy alone first, now and then (the in-flight bound waits on it)
  switch (r.below(3)) {
    case 0:
      check(sh_loader_sync_copy(L, ld.ticket) == SH_OK, "sh_loader_sync_copy", ld.kind);
      break;
    case 1: {
      int st;
      while ((st = sh_loader_query_copy(L, ld.ticket)) == SH_ERR_NOT_READY) std::this_thread::yield();
      check(st == SH_OK, "sh_loader_query_copy", ld.kind);
      break;
    }
    default:
      break;
  }
  switch (r.below(4)) {
    case 0: {
      int st;
      while ((st = sh_loader_query(L, ld.ticket)) == SH_ERR_NOT_READY) std::this_thread::yield();
      check(st == SH_OK, "sh_loader_query", ld.kind);
      break;
    }
    case 1:
      check(sh_loader_stream_wait(L, ld.ticket, s) == SH_OK, "sh_loader_stream_wait", ld.kind);
      check(hipStreamSynchronize(s) == hipSuccess, "hipStreamSynchronize");
      break;
    case 2:
      check(sh_loader_sync(L, ld.ticket) == SH_OK, "sh_loader_sync", ld.kind);
      break;
    default:
      check(sh_loader_release(L, ld.ticket) == SH_OK, "sh_loader_release (no wait)", ld.kind);
      released = true;
  }
  if (ld.bytes > 0) check(std::memcmp(ld.dst, ld.want.data(), ld.bytes) == 0, "loaded bytes", ld.kind);
  if (ld.digest != nullptr) {
    const uint64_t n = (ld.bytes + ld.chunk - 1) / ld.chunk;
    std::vector<uint64_t> want(2 * n);
    check(sh_block_digest_host(ld.want.data(), ld.bytes, ld.chunk, want.data()) == SH_OK, "host digest");
    check(std::memcmp(ld.digest, want.data(), 16 * n) == 0, "load digests");
  }
  if (!released) check(sh_loader_release(L, ld.ticket) == SH_OK, "sh_loader_release", ld.kind);
  if (ld.sb_ticket != 0) check(sh_saveback_release(sb, ld.sb_ticket) == SH_OK, "sh_saveback_release (load)");
  (void)hipFree(ld.dst);
  (void)hipFree(ld.dev_src);
  (void)hipFree(ld.digest);
  (void)hipHostFree(ld.pinned);
}

void loader_thread(sh_pool* pool, const std::string& path, const std::vector<uint8_t>& file, uint32_t seed,
                   int rounds) {
  Rng r(seed);
  sh_loader* L = nullptr;
  sh_saveback* sb = nullptr;
  check(sh_loader_create(pool, 4, &L) == SH_OK, "sh_loader_create");
  check(sh_saveback_create(0, &sb) == SH_OK, "sh_saveback_create");
  sh_file* f = nullptr;
  check(sh_file_open(path.c_str(), 0, &f) == SH_OK, "sh_file_open");
  hipStream_t s = nullptr;
  check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking) == hipSuccess, "hipStreamCreateWithFlags");
  if (!L || !sb || !f) return;
  std::deque<Load> pend;
  for (int round = 0; round < rounds; ++round) {
    Load ld;
    ld.kind = (int)r.below(5);
    ld.bytes = ld.kind == 0 ? 0 : 1 + r.below(3u << 20);
    ld.src.resize(ld.bytes);
    fill(ld.src, r);
    ld.want = ld.src;
    sh_load_request req{};
    sh_copy_item pieces[3];
    sh_copy_item dma{};
    sh_file_range range{};
    req.src_bytes = ld.bytes;
    req.scale_off = -1;
    req.zp_off = -1;
    if (ld.kind == 1 || ld.kind == 4) {  // host pieces at odd cuts
      const uint64_t a = ld.bytes / 3, b = ld.bytes - ld.bytes / 5;
      const uint64_t cuts[4] = {0, a, b, ld.bytes};
      for (int i = 0; i < 3; ++i)
        pieces[i] = {(void*)(uintptr_t)cuts[i], ld.src.data() + cuts[i], cuts[i + 1] - cuts[i]};
      req.pieces = pieces;
      req.n_pieces = 3;
    } else if (ld.kind == 2) {  // a file range
      ld.bytes = std::min<uint64_t>(ld.bytes, file.size() - 4096);
      const uint64_t off = r.below(file.size() - ld.bytes);
      ld.want.assign(file.begin() + (long)off, file.begin() + (long)(off + ld.bytes));
      range = {f, off, ld.bytes, 0};
      req.ranges = &range;
      req.n_ranges = 1;
      req.src_bytes = ld.bytes;
    } else if (ld.kind == 3) {  // pinned pieces that a save-back writes first
      ld.dev_src = dmalloc(ld.bytes);
      check(hipMemcpy(ld.dev_src, ld.src.data(), ld.bytes, hipMemcpyHostToDevice) == hipSuccess, "hipMemcpy");
      ld.pinned = hmalloc(ld.bytes);
      sh_copy_item it{ld.pinned, ld.dev_src, ld.bytes};
      check(sh_saveback_submit(sb, &it, 1, s, &ld.sb_ticket) == SH_OK, "sh_saveback_submit (load)");
      dma = {(void*)0, ld.pinned, ld.bytes};
      req.dma = &dma;
      req.n_dma = 1;
      req.saveback = sb;
      req.saveback_ticket = ld.sb_ticket;
    }
    if (ld.kind == 4) {
      const uint64_t n = (ld.bytes + ld.chunk - 1) / ld.chunk;
      ld.digest = (uint64_t*)dmalloc(16 * n);
      req.digest = ld.digest;
      req.digest_bytes = ld.bytes;
      req.digest_chunk = ld.chunk;
    }
    ld.dst = ld.bytes ? dmalloc(ld.bytes) : nullptr;
    req.dst = ld.dst;
    req.dst_bytes = ld.bytes;
    req.copy_threads = (int32_t)(1 + r.below(4));
    if (sh_loader_submit(L, &req, s, &ld.ticket) != SH_OK) {
      check(false, "sh_loader_submit", ld.kind);
      continue;
    }
    pend.push_back(std::move(ld));
    while (pend.size() > 3 || (!pend.empty() && r.below(3) == 0)) {
      const size_t k = r.below(pend.size());
      finish_load(L, sb, s, pend[k], r);
      pend.erase(pend.begin() + (long)k);
    }
  }
  while (!pend.empty()) {
    finish_load(L, sb, s, pend.front(), r);
    pend.pop_front();
  }
  check(sh_loader_destroy(L) == SH_OK, "sh_loader_destroy");
  check(sh_saveback_destroy(sb) == SH_OK, "sh_saveback_destroy");
  check(sh_file_close(f) == SH_OK, "sh_file_close");
  check(hipStreamDestroy(s) == hipSuccess, "hipStreamDestroy");
}

// ── save-back engine ──────────────────────────────────────────────────────

struct Copy {
  uint64_t ticket = 0;
  std::vector<uint8_t> want;
  std::vector<uint8_t> staging;  // the host bytes the device buffer was filled from
  void* dev = nullptr;
  void* host = nullptr;
  uint64_t* digests = nullptr;
  uint8_t* changed = nullptr;
  uint64_t expect_copied = UINT64_MAX;
  hipEvent_t ev = nullptr;
};

void saveback_stress(uint32_t seed, int rounds) {
  Rng r(seed);
  sh_saveback* sb = nullptr;
  check(sh_saveback_create(0, &sb) == SH_OK, "sh_saveback_create");
  hipStream_t s = nullptr;
  check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking) == hipSuccess, "hipStreamCreateWithFlags");
  if (!sb) return;
  std::mutex mu;
  std::deque<Copy*> queue;
  std::atomic<bool> done{false};

  std::thread consumer([&] {
    Rng rc(seed ^ 0x5555);
    std::vector<Copy*> held;
    auto finish = [&](Copy* c) {
      check(sh_saveback_wait(sb, c->ticket) == SH_OK, "sh_saveback_wait");
      if (!c->want.empty()) check(std::memcmp(c->host, c->want.data(), c->want.size()) == 0, "saved-back bytes");
      if (c->expect_copied != UINT64_MAX) {
        uint64_t got = 0;
        check(sh_saveback_ticket_bytes(sb, c->ticket, &got) == SH_OK && got == c->expect_copied,
              "changed-chunk bytes", (long)got);
      }
      check(sh_saveback_release(sb, c->ticket) == SH_OK, "sh_saveback_release");
      check(sh_saveback_release(sb, c->ticket) == SH_OK, "second release is a no-op");
      (void)hipFree(c->dev);
      (void)hipFree(c->digests);
      (void)hipHostFree(c->host);
      (void)hipHostFree(c->changed);
      if (c->ev) (void)hipEventDestroy(c->ev);
      delete c;
    };
    for (;;) {
      Copy* c = nullptr;
      {
        std::lock_guard<std::mutex> lk(mu);
        if (!queue.empty()) {
          c = queue.front();
          queue.pop_front();
        }
      }
      if (c == nullptr) {
        if (done.load() && held.empty()) break;
        if (!held.empty()) {  // later tickets first, then the earlier ones
          for (auto it = held.rbegin(); it != held.rend(); ++it) finish(*it);
          held.clear();
        }
        std::this_thread::yield();
        continue;
      }
      held.push_back(c);
      if (held.size() > 2 + rc.below(3)) {
        for (auto it = held.rbegin(); it != held.rend(); ++it) finish(*it);
        held.clear();
      }
    }
  });

  for (int round = 0; round < rounds; ++round) {
    Copy* c = new Copy();
    const int kind = (int)r.below(4);
    const uint64_t bytes = kind == 0 ? 0 : 16 + r.below(1u << 20);
    c->staging.resize(bytes);
    fill(c->staging, r);
    c->want = c->staging;
    if (bytes) {
      c->dev = dmalloc(bytes);
      c->host = hmalloc(bytes);
      check(hipMemcpyAsync(c->dev, c->staging.data(), bytes, hipMemcpyHostToDevice, s) == hipSuccess,
            "hipMemcpyAsync (fill)");
    }
    sh_copy_item it{c->host, c->dev, bytes};
    int st = SH_OK;
    if (kind == 0) {
      st = sh_saveback_submit(sb, nullptr, 0, s, &c->ticket);
    } else if (kind == 1) {
      st = sh_saveback_submit(sb, &it, 1, s, &c->ticket);
    } else if (kind == 2) {
      check(hipEventCreateWithFlags(&c->ev, hipEventDisableTiming) == hipSuccess, "hipEventCreate");
      check(hipEventRecord(c->ev, s) == hipSuccess, "hipEventRecord");
      void* evs[1] = {c->ev};
      st = sh_saveback_submit_after(sb, &it, 1, evs, 1, &c->ticket);
    } else {
      // changed chunks: the home buffer holds the bytes, the device changes two chunks
      const uint32_t chunk = 4096;
      const uint64_t n = (bytes + chunk - 1) / chunk;
      check(hipStreamSynchronize(s) == hipSuccess, "hipStreamSynchronize");
      std::memcpy(c->host, c->staging.data(), bytes);
      c->digests = (uint64_t*)dmalloc(16 * n);
      c->changed = (uint8_t*)hmalloc(n);
      check(sh_block_digest(c->dev, bytes, chunk, c->digests, s) == SH_OK, "sh_block_digest");
      std::vector<uint64_t> touched;
      for (int k = 0; k < 2; ++k) {
        const uint64_t at = r.below(bytes);
        c->want[at] ^= 0x5A;
        touched.push_back(at / chunk);
        check(hipMemcpyAsync((uint8_t*)c->dev + at, c->want.data() + at, 1, hipMemcpyHostToDevice, s) == hipSuccess,
              "hipMemcpyAsync (change)");
      }
      std::sort(touched.begin(), touched.end());
      touched.erase(std::unique(touched.begin(), touched.end()), touched.end());
      c->expect_copied = 0;
      for (uint64_t t : touched) c->expect_copied += std::min<uint64_t>(chunk, bytes - t * chunk);
      sh_chunk_region reg{c->host, c->dev, bytes, 0};
      st = sh_saveback_submit_chunks(sb, &reg, 1, chunk, c->digests, c->changed, s, nullptr, 0, s, &c->ticket);
    }
    check(st == SH_OK, "save-back submit", kind);
    {
      std::lock_guard<std::mutex> lk(mu);
      queue.push_back(c);
    }
    if (r.below(16) == 0) std::this_thread::sleep_for(std::chrono::microseconds(200));
  }
  done.store(true);
  consumer.join();
  // destroy with copies still queued: it issues and waits for them
  std::vector<uint8_t> src(1 << 20, 7);
  void* dev = dmalloc(src.size());
  void* host = hmalloc(src.size());
  check(hipMemcpyAsync(dev, src.data(), src.size(), hipMemcpyHostToDevice, s) == hipSuccess, "fill");
  sh_copy_item it{host, dev, src.size()};
  uint64_t t = 0;
  check(sh_saveback_submit(sb, &it, 1, s, &t) == SH_OK, "last submit");
  check(sh_saveback_destroy(sb) == SH_OK, "sh_saveback_destroy with a queued ticket");
  check(std::memcmp(host, src.data(), src.size()) == 0, "bytes of the ticket queued at destroy");
  (void)hipFree(dev);
  (void)hipHostFree(host);
  check(hipStreamDestroy(s) == hipSuccess, "hipStreamDestroy");
}

// ── turbo engine ──────────────────────────────────────────────────────────

void turbo_stress(uint32_t seed) {
  Rng r(seed);
  constexpr uint32_t kBlocks = 6, kWindow = 3;
  std::vector<std::vector<std::vector<uint8_t>>> data(kBlocks);
  sh_turbo* t = nullptr;
  check(sh_turbo_create(&t) == SH_OK, "sh_turbo_create");
  if (!t) return;
  for (uint32_t b = 0; b < kBlocks; ++b) {
    const uint64_t sizes[3] = {3000 + 512 * b, 70000, 123};
    for (uint64_t n : sizes) {
      data[b].emplace_back(n);
      fill(data[b].back(), r);
    }
    uint32_t idx = 0;
    check(sh_turbo_register_block(t, sizes, 3, &idx) == SH_OK && idx == b, "sh_turbo_register_block");
  }
  check(sh_turbo_set_save_back(t, 1) == SH_OK, "sh_turbo_set_save_back");
  check(sh_turbo_set_writeback_chunks(t, 4096) == SH_OK, "sh_turbo_set_writeback_chunks");
  check(sh_turbo_initialize(t, 0, kWindow) == SH_OK, "sh_turbo_initialize");
  for (uint32_t b = 0; b < kBlocks; ++b) {
    const void* src[3] = {data[b][0].data(), data[b][1].data(), data[b][2].data()};
    check(sh_turbo_stage_block(t, b, src, 3) == SH_OK, "sh_turbo_stage_block");
  }
  uint64_t slot_bytes = 0;
  check(sh_turbo_slot_bytes(t, &slot_bytes) == SH_OK, "sh_turbo_slot_bytes");
  std::vector<uint8_t*> slots;
  for (uint32_t s = 0; s < kWindow; ++s) {
    slots.push_back((uint8_t*)dmalloc(slot_bytes));
    check(sh_turbo_set_slot_buffer(t, s, slots.back(), slot_bytes) == SH_OK, "sh_turbo_set_slot_buffer");
  }
  hipStream_t cs = nullptr;
  check(hipStreamCreateWithFlags(&cs, hipStreamNonBlocking) == hipSuccess, "hipStreamCreateWithFlags");
  uint8_t* bump = (uint8_t*)hmalloc(4096);  // the "optimizer" values written on the compute stream
  int bump_i = 0;

  auto verify_on_device = [&](uint32_t b) {
    int32_t slot = -1;
    check(sh_turbo_block_slot(t, b, &slot) == SH_OK && slot >= 0, "sh_turbo_block_slot", b);
    if (slot < 0) return;
    check(hipStreamSynchronize(cs) == hipSuccess, "sync");
    check(hipDeviceSynchronize() == hipSuccess, "the block's H2D has landed");
    for (uint32_t p = 0; p < 3; ++p) {
      uint64_t off = 0;
      check(sh_turbo_param_offset(t, b, p, &off) == SH_OK, "sh_turbo_param_offset");
      check(std::memcmp(slots[slot] + off, data[b][p].data(), data[b][p].size()) == 0, "slot bytes", b * 10 + p);
    }
  };
  auto step_and_change = [&](uint32_t b, int dir) -> int {
    const int st = sh_turbo_step(t, b, dir, cs);
    if (st != SH_OK) return st;
    int32_t slot = -1;
    check(sh_turbo_block_slot(t, b, &slot) == SH_OK && slot >= 0, "block slot after step", b);
    if (slot < 0) return SH_OK;
    // change one byte of param 0 and one of param 1 on the compute stream, as training would
    // (a failure armed for the engine's copies stays armed for them, not for these)
    const int armed = fake_hip_fail_pending("hipMemcpyAsync");
    fake_hip_fail_next("hipMemcpyAsync", 0);
    for (uint32_t p = 0; p < 2; ++p) {
      uint64_t off = 0;
      (void)sh_turbo_param_offset(t, b, p, &off);
      const uint64_t at = r.below(data[b][p].size());
      const uint8_t v = (uint8_t)(data[b][p][at] + 1);
      data[b][p][at] = v;
      uint8_t* src = bump + (bump_i++ % 4096);
      check(hipStreamSynchronize(cs) == hipSuccess, "sync before reusing the bump byte");
      *src = v;
      check(hipMemcpyAsync(slots[slot] + off + at, src, 1, hipMemcpyHostToDevice, cs) == hipSuccess, "change");
    }
    fake_hip_fail_next("hipMemcpyAsync", armed);
    return SH_OK;
  };

  fake_hip_sdma_delay_us(3000);  // write-backs slower than a step: look-ahead copies get deferred
  for (int round = 0; round < 2; ++round) {
    for (uint32_t b = 0; b < kBlocks; ++b) check(step_and_change(b, SH_TURBO_FORWARD) == SH_OK, "forward step", b);
    for (uint32_t b = kBlocks; b-- > 0;) check(step_and_change(b, SH_TURBO_BACKWARD) == SH_OK, "backward step", b);
  }
  // H2D copies that fail, armed at points of a forward and a backward pass while look-ahead copies
  // are being deferred behind slow write-backs: the step reports the failure, no block keeps a
  // slot it was not loaded into, and the step tried again loads the block with its bytes.
  auto invariants = [&](long where) {
    uint32_t nb = 0, ns = 0, nfree = 0, assigned = 0;
    check(sh_turbo_counts(t, &nb, &ns, &nfree) == SH_OK, "sh_turbo_counts");
    for (uint32_t k = 0; k < kBlocks; ++k) {
      int32_t slot = -1;
      int loc = -1;
      (void)sh_turbo_block_slot(t, k, &slot);
      (void)sh_turbo_block_location(t, k, &loc);
      assigned += slot >= 0;
      check((slot >= 0) == (loc == SH_TURBO_GPU || loc == SH_TURBO_H2D), "a slot exactly when on the device",
            where * 10 + k);
    }
    check(nfree + assigned == ns, "every slot is free or held by one block", where);
  };
  int failed_steps = 0;
  for (int round = 0; round < 3; ++round) {
    for (int dir : {SH_TURBO_FORWARD, SH_TURBO_BACKWARD}) {
      for (uint32_t k = 0; k < kBlocks; ++k) {
        const uint32_t b = dir == SH_TURBO_FORWARD ? k : kBlocks - 1 - k;
        if (k == 1 + (uint32_t)round) fake_hip_fail_next("hipMemcpyAsync", 1);
        int st = step_and_change(b, dir);
        if (st != SH_OK) {
          ++failed_steps;
          check(fake_hip_fail_pending("hipMemcpyAsync") == 0, "only the injected failure", b);
          invariants(b);
          st = step_and_change(b, dir);
        }
        check(st == SH_OK, "step after an injected failure", b);
        verify_on_device(b);
      }
    }
    fake_hip_fail_next("hipMemcpyAsync", 0);
  }
  check(failed_steps >= 3, "the injected copy failures were reported", failed_steps);
  check(hipStreamSynchronize(cs) == hipSuccess, "sync");
  check(sh_turbo_drain(t) == SH_OK, "sh_turbo_drain");
  fake_hip_sdma_delay_us(0);
  for (uint32_t b = 0; b < kBlocks; ++b) {
    int loc = -1;
    check(sh_turbo_block_location(t, b, &loc) == SH_OK, "sh_turbo_block_location");
    if (loc != SH_TURBO_CPU) continue;
    for (uint32_t p = 0; p < 3; ++p) {
      uint64_t ptr = 0;
      check(sh_turbo_cpu_ptr(t, b, p, &ptr) == SH_OK, "sh_turbo_cpu_ptr");
      check(std::memcmp((void*)(uintptr_t)ptr, data[b][p].data(), data[b][p].size()) == 0, "written-back bytes",
            b * 10 + p);
    }
  }
  check(sh_turbo_destroy(t) == SH_OK, "sh_turbo_destroy");
  for (uint8_t* s : slots) (void)hipFree(s);
  (void)hipHostFree(bump);
  check(hipStreamDestroy(cs) == hipSuccess, "hipStreamDestroy");
}

// ── VMM allocator ─────────────────────────────────────────────────────────

void vmm_stress(uint32_t seed, int iters) {
  constexpr uint64_t kRegion = 64 << 10;
  constexpr uint32_t kRegions = 8;
  sh_vmm* v = nullptr;
  check(sh_vmm_create(0, 4 * kRegion, &v) == SH_OK, "sh_vmm_create");
  if (!v) return;
  uint32_t slab = 0;
  check(sh_vmm_create_slab(v, kRegions * kRegion, &slab) == SH_OK, "sh_vmm_create_slab");
  for (uint32_t i = 0; i < kRegions; ++i) {
    uint32_t id = 0;
    check(sh_vmm_define_region(v, slab, i * kRegion, kRegion, &id) == SH_OK && id == i, "sh_vmm_define_region");
  }
  check(sh_vmm_set_priority(v, slab, 1) == SH_OK, "sh_vmm_set_priority");
  std::atomic<int> served{0}, refused{0};
  std::atomic<bool> stop{false};
  auto user = [&](uint32_t tid) {
    Rng r(seed * 31 + tid);
    hipStream_t s = nullptr;
    check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking) == hipSuccess, "hipStreamCreateWithFlags");
    for (int k = 0; k < iters; ++k) {
      const uint32_t region = (uint32_t)r.below(kRegions);
      sh_vmm_handle* h = nullptr;
      const int st = sh_vmm_ensure_resident(v, slab, region, s, &h);
      if (st == SH_ERR_WATERMARK) {
        refused.fetch_add(1);
        // the watermark falls to an evicted region; the highest-priority slab re-opens it
        check(sh_vmm_set_priority(v, slab, 1) == SH_OK, "re-open the watermark");
        continue;
      }
      check(st == SH_OK, "sh_vmm_ensure_resident", st);
      if (st != SH_OK) continue;
      void* p = nullptr;
      check(sh_vmm_handle_ptr(h, &p) == SH_OK && p != nullptr, "sh_vmm_handle_ptr");
      // the region stays mapped while the handle is held: write and read a stamp at a spot of this thread's own
      uint8_t* b = (uint8_t*)p + 64 * tid;
      const uint8_t stamp = (uint8_t)(k * 7 + tid);
      for (int i = 0; i < 64; ++i) b[i] = stamp;
      std::this_thread::yield();
      for (int i = 0; i < 64; ++i) check(b[i] == stamp, "region bytes while held", region);
      served.fetch_add(1);
      check(sh_vmm_handle_release(h) == SH_OK, "sh_vmm_handle_release");
      check(sh_vmm_handle_release(h) == SH_ERR_STATE, "a second release is refused");
      check(sh_vmm_handle_destroy(h) == SH_OK, "sh_vmm_handle_destroy");
    }
    check(hipStreamSynchronize(s) == hipSuccess, "sync");
    check(hipStreamDestroy(s) == hipSuccess, "hipStreamDestroy");
  };
  std::thread side([&] {
    Rng r(seed ^ 0xABC);
    while (!stop.load()) {
      (void)sh_vmm_prefetch(v, slab, (uint32_t)r.below(kRegions));
      sh_vmm_stats st{};
      check(sh_vmm_info(v, &st) == SH_OK, "sh_vmm_info");
      check(st.mapped_bytes <= 4 * kRegion + kRegion, "mapped bytes stay near the ceiling", (long)st.mapped_bytes);
      sh_vmm_region_stats rs{};
      check(sh_vmm_region_info(v, slab, (uint32_t)r.below(kRegions), &rs) == SH_OK, "sh_vmm_region_info");
      std::this_thread::yield();
    }
  });
  std::vector<std::thread> users;
  for (uint32_t tid = 0; tid < 3; ++tid) users.emplace_back(user, tid);
  for (std::thread& u : users) u.join();
  stop.store(true);
  side.join();
  sh_vmm_stats st{};
  check(sh_vmm_info(v, &st) == SH_OK && st.evictions > 0, "regions were evicted under the ceiling",
        (long)st.evictions);
  check(served.load() > 0, "regions were served");
  check(sh_vmm_destroy_slab(v, slab) == SH_OK, "sh_vmm_destroy_slab");
  check(sh_vmm_destroy(v) == SH_OK, "sh_vmm_destroy");
  std::fprintf(stderr, "vmm: %d served, %d refused at the watermark, %llu evictions\n", served.load(),
               refused.load(), (unsigned long long)st.evictions);
}

}  // namespace

int main() {
  // a weight file for the loader's file ranges
  char path[] = "/tmp/sh_engine_stress_XXXXXX";
  const int fd = mkstemp(path);
  if (fd < 0) return 2;
  std::vector<uint8_t> file(6u << 20);
  Rng fr(99);
  fill(file, fr);
  if (write(fd, file.data(), file.size()) != (ssize_t)file.size()) return 2;
  close(fd);

  sh_pool* pool = nullptr;
  check(sh_pool_create(4, 1u << 20, 1, &pool) == SH_OK, "sh_pool_create");
  {
    std::vector<std::thread> ts;
    ts.emplace_back(loader_thread, pool, std::string(path), std::cref(file), 1u, 60);
    ts.emplace_back(loader_thread, pool, std::string(path), std::cref(file), 2u, 60);
    ts.emplace_back(saveback_stress, 3u, 120);
    ts.emplace_back(vmm_stress, 4u, 400);
    for (std::thread& t : ts) t.join();
  }
  turbo_stress(5);
  check(sh_pool_destroy(pool) == SH_OK, "sh_pool_destroy");
  sh_live_counts live{};
  check(sh_shutdown(&live) == SH_OK, "sh_shutdown");
  check(live.loaders == 0 && live.savebacks == 0 && live.turbos == 0 && live.vmms == 0 && live.pools == 0,
        "every engine destroyed");
  unlink(path);
  std::printf("engine_stress: ok (%d failures)\n", g_failures.load());
  return g_failures.load() == 0 ? 0 : 1;
}
