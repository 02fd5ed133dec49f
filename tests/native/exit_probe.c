/* Lists what libstagehand_native.so leaves to the process's exit (tests/test_exit_handlers.py
 * builds and runs this on the CPU).
 *
 * The program defines __cxa_atexit and __cxa_thread_atexit_impl itself and exports them
 * (-rdynamic), so every registration the library makes (its static destructors, atexit calls,
 * compiler-emitted module destructors, C++ thread_local destructors) comes here first. Each is
 * logged with the module its handler lives in and passed on to libc. The program loads the
 * library, drives the entry points that run without a GPU (plans, host copies on the shared
 * copy threads, file reads, the host digest, the pool, the allocation-free entry point up to
 * its device lookup), on the main thread and on a second thread, calls sh_shutdown and exits.
 * A destructor of this program runs after every exit handler has run, so it also sees anything
 * registered during the exit itself: its line says how many handlers belong to the library,
 * and the program then ends with status 3 if any does. */
#define _GNU_SOURCE
#include <dlfcn.h>
#include <fcntl.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "stagehand_native.h"

static int g_lib_handlers = 0;

static int from_library(const void* addr) {
  Dl_info info;
  memset(&info, 0, sizeof info);
  if (dladdr(addr, &info) == 0 || info.dli_fname == NULL) return 0;
  return strstr(info.dli_fname, "libstagehand_native") != NULL;
}

static void note(const char* kind, void (*fn)(void*), void* dso) {
  Dl_info info;
  memset(&info, 0, sizeof info);
  dladdr((void*)fn, &info);
  const int mine = from_library((void*)fn) || (dso != NULL && from_library(dso));
  if (mine) {
    ++g_lib_handlers;
    fprintf(stderr, "exit_probe: library handler %s fn=%s+0x%lx (%s)\n", kind,
            info.dli_fname ? info.dli_fname : "?", (unsigned long)((char*)fn - (char*)info.dli_fbase),
            info.dli_sname ? info.dli_sname : "no symbol");
  }
}

int __cxa_atexit(void (*fn)(void*), void* arg, void* dso) {
  static int (*real)(void (*)(void*), void*, void*);
  if (real == NULL) real = (int (*)(void (*)(void*), void*, void*))dlsym(RTLD_NEXT, "__cxa_atexit");
  note("__cxa_atexit", fn, dso);
  return real(fn, arg, dso);
}

int __cxa_thread_atexit_impl(void (*fn)(void*), void* obj, void* dso) {
  static int (*real)(void (*)(void*), void*, void*);
  if (real == NULL) real = (int (*)(void (*)(void*), void*, void*))dlsym(RTLD_NEXT, "__cxa_thread_atexit_impl");
  note("__cxa_thread_atexit_impl", fn, dso);
  return real(fn, obj, dso);
}

static int g_failures = 0;
static void expect(int ok, const char* what) {
  if (!ok) {
    fprintf(stderr, "exit_probe: FAIL %s (%s)\n", what, sh_last_error());
    ++g_failures;
  }
}

static const char* g_path;

/* What the block loader's host staging does without a GPU. */
static void* host_work(void* arg) {
  (void)arg;
  enum { kBytes = 3 << 20 };
  uint8_t* src = (uint8_t*)malloc(kBytes);
  uint8_t* dst = (uint8_t*)malloc(kBytes + 4096);
  for (size_t i = 0; i < kBytes; ++i) src[i] = (uint8_t)(i * 131u >> 3);
  sh_copy_item items[2] = {{dst, src, kBytes / 2}, {dst + kBytes / 2, src + kBytes / 2, kBytes - kBytes / 2}};
  expect(sh_host_copy_batch(items, 2, 4) == SH_OK && memcmp(dst, src, kBytes) == 0, "sh_host_copy_batch");

  uint64_t dg[2 * 4];
  expect(sh_block_digest_host(src, kBytes, 1u << 20, dg) == SH_OK, "sh_block_digest_host");

  for (int flags = 0; flags <= SH_FILE_DIRECT; flags += SH_FILE_DIRECT) {
    sh_file* f = NULL;
    expect(sh_file_open(g_path, flags, &f) == SH_OK, "sh_file_open");
    if (f != NULL) {
      /* destination 16 bytes past an aligned address: not congruent to the file offset, so a
       * direct read goes through the thread's bounce buffer */
      sh_file_range r = {f, 4096, kBytes - 8192, 16};
      memset(dst, 0, kBytes);
      expect(sh_file_read_batch(&r, 1, dst, 4) == SH_OK && memcmp(dst + 16, src + 4096, kBytes - 8192) == 0,
             "sh_file_read_batch");
      expect(sh_file_close(f) == SH_OK, "sh_file_close");
    }
  }
  free(src);
  free(dst);
  return NULL;
}

int main(int argc, char** argv) {
  if (argc < 2) {
    fprintf(stderr, "usage: exit_probe <scratch file>\n");
    return 2;
  }
  g_path = argv[1];
  expect(sh_abi_version() == SH_ABI_VERSION, "sh_abi_version");

  /* the scratch file the reads use: the same bytes host_work copies */
  {
    enum { kBytes = 3 << 20 };
    uint8_t* buf = (uint8_t*)malloc(kBytes);
    for (size_t i = 0; i < kBytes; ++i) buf[i] = (uint8_t)(i * 131u >> 3);
    FILE* fp = fopen(g_path, "wb");
    expect(fp != NULL && fwrite(buf, 1, kBytes, fp) == kBytes, "writing the scratch file");
    if (fp) fclose(fp);
    free(buf);
  }

  sh_unpack_desc d[2];
  memset(d, 0, sizeof d);
  d[0].src_off = 8; d[0].dst_off = 0; d[0].rows = 96; d[0].cols = 3072; d[0].kind = SH_KIND_I8_ROWSCALE_BF16;
  d[1].src_off = 8 + 96 * 3072; d[1].dst_off = 2 * 96 * 3072; d[1].rows = 1; d[1].cols = 96; d[1].kind = SH_KIND_F32_BF16;
  sh_plan_info info;
  expect(sh_plan_describe(d, 2, &info) == SH_OK && info.n_desc == 2, "sh_plan_describe");
  /* fails at its device lookup here (no GPU), after it has built its table */
  (void)sh_unpack_noalloc(d, 2, (void*)64, 1 << 20, (const float*)64, NULL, 96, (void*)64, 1 << 20, NULL);

  sh_pool* pool = NULL;
  expect(sh_pool_create(3, 1 << 16, 0, &pool) == SH_OK, "sh_pool_create");
  uint32_t slab = 0;
  double waited = 0;
  expect(pool != NULL && sh_pool_acquire(pool, 1000, &slab, &waited) == SH_OK, "sh_pool_acquire");
  expect(pool != NULL && sh_pool_release(pool, slab) == SH_OK, "sh_pool_release");
  expect(sh_pool_destroy(pool) == SH_OK, "sh_pool_destroy");

  host_work(NULL);
  pthread_t t;
  expect(pthread_create(&t, NULL, host_work, NULL) == 0, "pthread_create");
  pthread_join(t, NULL);

  sh_live_counts live;
  memset(&live, 0xff, sizeof live);
  expect(sh_shutdown(&live) == SH_OK, "sh_shutdown");
  expect(live.pools == 0 && live.files == 0 && live.copy_threads == 0 && live.kernel_devices == 0,
         "nothing alive after sh_shutdown");
  unlink(g_path);
  printf("exit_probe: %d failures\n", g_failures);
  fflush(stdout);
  return g_failures == 0 ? 0 : 1;
}

__attribute__((destructor)) static void report(void) {
  printf("exit_probe: %d library exit handlers\n", g_lib_handlers);
  fflush(stdout);
  if (g_lib_handlers != 0) _exit(3);
}
