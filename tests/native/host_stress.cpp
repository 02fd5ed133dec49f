// Multi-threaded stress of the library's host-side native code, built with the thread and
// address sanitizers (Makefile in this directory; tests/test_sanitizers.py runs it on the CPU).
//
// It drives, from several threads at once, what the block loader does on its copy threads
// without a GPU: the pinned-slab pool's acquire/release/stats (unpinned memory), host copy
// batches and weight-file read batches on the shared copy threads (run_io), thread-local
// error reporting, and sh_shutdown joining the copy threads while another thread still
// copies. Every byte copied or read is checked; any mismatch exits non-zero, and the
// sanitizers exit non-zero on a race, an out-of-bounds access or undefined behaviour.

#include <unistd.h>

#include <atomic>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "stagehand_native.h"

namespace {

std::atomic<int> g_failures{0};

void check(bool ok, const char* what) {
  if (!ok) {
    std::fprintf(stderr, "FAIL: %s (last error: %s)\n", what, sh_last_error());
    g_failures.fetch_add(1);
  }
}

uint8_t pattern(uint64_t i, uint32_t seed) { return (uint8_t)((i * 2654435761u) >> 13 ^ seed); }

void pool_stress(sh_pool* pool, uint32_t seed, int rounds) {
  for (int r = 0; r < rounds; ++r) {
    uint32_t slab = 0;
    double waited = 0;
    if (sh_pool_acquire(pool, 5000, &slab, &waited) != SH_OK) {
      check(false, "sh_pool_acquire");
      return;
    }
    void* p = nullptr;
    check(sh_pool_slab_ptr(pool, slab, &p) == SH_OK && p != nullptr, "sh_pool_slab_ptr");
    std::memset(p, (int)(seed + r), 4096);  // the slab is ours until released
    sh_pool_stats st{};
    check(sh_pool_get_stats(pool, &st) == SH_OK && st.in_use >= 1 && st.in_use <= st.total, "pool stats");
    check(((uint8_t*)p)[4095] == (uint8_t)(seed + r), "slab contents while held");
    check(sh_pool_release(pool, slab) == SH_OK, "sh_pool_release");
  }
}

void copy_stress(uint32_t seed, int rounds, size_t bytes) {
  std::vector<uint8_t> src(bytes), dst(bytes + 64);
  for (size_t i = 0; i < bytes; ++i) src[i] = pattern(i, seed);
  for (int r = 0; r < rounds; ++r) {
    // three items at odd offsets and lengths, one of them empty
    const size_t a = bytes / 3 + 7, b = bytes - a - 5;
    sh_copy_item items[3] = {{dst.data() + 1, src.data(), a}, {dst.data() + 1 + a, src.data() + a, 0},
                             {dst.data() + 1 + a, src.data() + a, b}};
    check(sh_host_copy_batch(items, 3, 8) == SH_OK, "sh_host_copy_batch");
    check(std::memcmp(dst.data() + 1, src.data(), a + b) == 0, "copied bytes");
  }
}

void file_stress(const std::string& path, uint32_t seed, int rounds, size_t fsize) {
  sh_file* f = nullptr;
  if (sh_file_open(path.c_str(), 0, &f) != SH_OK) {
    check(false, "sh_file_open");
    return;
  }
  std::vector<uint8_t> buf(fsize + 4096);
  for (int r = 0; r < rounds; ++r) {
    // ranges out of order, crossing the 8 MiB piece size, landing at shifted offsets
    const uint64_t half = fsize / 2;
    sh_file_range ranges[2] = {{f, half, fsize - half, 3}, {f, 0, half, 3 + (fsize - half)}};
    check(sh_file_read_batch(ranges, 2, buf.data(), 8) == SH_OK, "sh_file_read_batch");
    bool ok = true;
    for (uint64_t i = 0; i < fsize - half && ok; i += 4093) ok = buf[3 + i] == pattern(half + i, 0);
    for (uint64_t i = 0; i < half && ok; i += 4093) ok = buf[3 + (fsize - half) + i] == pattern(i, 0);
    check(ok, "file bytes");
    // a range past the end of the file is refused, with this thread's own error text
    sh_file_range bad = {f, fsize - 8, 16, 0};
    check(sh_file_read_batch(&bad, 1, buf.data(), 2) == SH_ERR_INVALID, "range past EOF refused");
    check(std::strlen(sh_last_error()) > 0, "error text set");
    (void)seed;
  }
  sh_file_info info{};
  check(sh_file_get_info(f, &info) == SH_OK && info.size == fsize, "sh_file_get_info");
  check(sh_file_close(f) == SH_OK, "sh_file_close");
}

}  // namespace

int main() {
  const size_t fsize = (24u << 20) + 12345;  // three 8 MiB pieces and a ragged tail
  char path[] = "/tmp/sh_host_stress_XXXXXX";
  int fd = mkstemp(path);
  if (fd < 0) return 2;
  {
    std::vector<uint8_t> data(fsize);
    for (size_t i = 0; i < fsize; ++i) data[i] = pattern(i, 0);
    if (write(fd, data.data(), fsize) != (ssize_t)fsize) return 2;
    close(fd);
  }
  sh_pool* pool = nullptr;
  check(sh_pool_create(3, 1 << 20, /*pinned=*/0, &pool) == SH_OK, "sh_pool_create");

  std::vector<std::thread> ts;
  for (uint32_t t = 0; t < 6; ++t) ts.emplace_back(pool_stress, pool, t, 200);
  for (uint32_t t = 0; t < 3; ++t) ts.emplace_back(copy_stress, t + 10, 20, (size_t)(9u << 20) + 333);
  for (uint32_t t = 0; t < 3; ++t) ts.emplace_back(file_stress, std::string(path), t, 6, fsize);
  for (auto& t : ts) t.join();
  ts.clear();

  // sh_shutdown while another thread keeps copying: the copy threads are joined when that
  // thread's current batch returns, and the next batch starts new ones
  std::atomic<bool> stop{false};
  std::thread copier([&] {
    while (!stop.load()) copy_stress(99, 1, (size_t)(3u << 20) + 1);
  });
  for (int i = 0; i < 20; ++i) {
    sh_live_counts live{};
    check(sh_shutdown(&live) == SH_OK, "sh_shutdown (busy)");
    check(live.pools == 1 && live.files == 0, "live counts while busy");
    std::this_thread::sleep_for(std::chrono::milliseconds(2));
  }
  stop.store(true);
  copier.join();

  check(sh_pool_destroy(pool) == SH_OK, "sh_pool_destroy");
  sh_live_counts live{};
  check(sh_shutdown(&live) == SH_OK, "sh_shutdown");
  check(live.pools == 0 && live.loaders == 0 && live.files == 0 && live.copy_threads == 0, "nothing left");
  unlink(path);
  const int failures = g_failures.load();
  std::printf("host_stress: %s (%d failures)\n", failures ? "FAILED" : "ok", failures);
  return failures ? 1 : 0;
}
