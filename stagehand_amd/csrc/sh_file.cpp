// Weight-file reader: bulk pread (and O_DIRECT) of byte ranges into host
// memory on the shared copy threads.
//
// The reference reads file-backed parameters through an mmap, one tensor at a
// time (torch.frombuffer over the mapping, then copy_ into the pinned slab:
// src/stagehand/scheduler.py:184-241, 564-601), and the VMM backend fills
// regions from the same mapping after an madvise(WILLNEED)
// (src/stagehand/vmm_backend.py:283-291). Here a block's ranges become pread
// calls of at most 8 MiB, cut at 8 MiB file offsets and run in parallel: a
// hot file is copied out of the page cache by every copy thread, holding no
// mapping of it (copying from a mapping measured as fast). Buffered pieces are
// read in two phases: every thread first copies what the page cache already
// holds (preadv2 with RWF_NOWAIT), then the remainders, sorted by file and offset, are cut into up to kColdStreams
// contiguous runs of about equal size, each read front to back by one thread
// on a descriptor of its own, so that each run is a sequential stream to the
// kernel's read-ahead (which is kept per open file). Interleaved cold reads
// of one file defeat that read-ahead: measured on a virtio disk, cold 8 MiB
// pieces handed out to 16 threads on one descriptor read 3.3-4.9 GB/s, 4
// contiguous runs on 4 descriptors 6.9 GB/s, one run 6.5 GB/s (O_DIRECT 7.2).
//
// With SH_FILE_DIRECT an O_DIRECT descriptor is opened as well and every
// read goes around the page cache (neither read nor filled):
//  * a piece whose destination address is congruent to its file offset modulo
//    SH_FILE_ALIGN reads its aligned middle straight into the destination (the
//    storage DMA writes it) and its unaligned head and tail through the page
//    cache — when the kernel can pin the destination for DMA;
//  * otherwise the piece's aligned cover is read into a per-thread aligned
//    bounce buffer and copied out. Host memory from hipHostMalloc is mapped by
//    the GPU driver and cannot be pinned again for a DMA (the direct read
//    fails with EFAULT), so loads into pinned slabs take this route; the first
//    EFAULT switches the file to it.
// A file system that refuses O_DIRECT at open leaves the file buffered only;
// one that refuses a direct read (EINVAL) makes the file fall back to
// buffered reads from then on.

#include <errno.h>
#include <fcntl.h>
#include <pthread.h>
#include <sys/stat.h>
#include <sys/uio.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cstring>
#include <cstdlib>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "sh_internal.h"
#include "stagehand_native.h"

struct sh_file {
  sh::Live<sh::kLiveFile> live;
  int fd = -1;                    // buffered descriptor
  std::atomic<int> dfd{-1};       // O_DIRECT descriptor, -1 when unavailable
  int dfd_owned = -1;             // closed at sh_file_close even after a fallback
  uint64_t size = 0;
  std::string path;
  std::atomic<bool> dma_refused{false};  // a zero-copy direct read failed with EFAULT
  std::atomic<bool> nowait_refused{false};  // the file system refuses RWF_NOWAIT reads
  std::atomic<uint64_t> bytes_direct{0};
  std::atomic<uint64_t> bytes_bounced{0};
  std::atomic<uint64_t> bytes_buffered{0};
  std::atomic<uint64_t> bytes_cached{0};
  std::atomic<uint64_t> reads{0};
  // descriptors of the cold-read streams (stream 0 reads on fd); opened on first use
  std::mutex stream_mu;
  int stream_fd[4] = {-1, -1, -1, -1};
};

namespace {

constexpr uint64_t kPiece = 8ull << 20;  // read / copy granule per thread
constexpr uint64_t kAlign = SH_FILE_ALIGN;

// pread until `bytes` are read; returns 0 or the errno of the failure
// (ENODATA for an unexpected end of file).
int pread_full(sh_file* f, int fd, uint8_t* dst, uint64_t off, uint64_t bytes) {
  while (bytes > 0) {
    const size_t want = (size_t)std::min<uint64_t>(bytes, 1ull << 30);
    const ssize_t r = ::pread(fd, dst, want, (off_t)off);
    f->reads.fetch_add(1, std::memory_order_relaxed);
    if (r < 0) {
      if (errno == EINTR) continue;
      return errno;
    }
    if (r == 0) return ENODATA;
    dst += r;
    off += (uint64_t)r;
    bytes -= (uint64_t)r;
  }
  return 0;
}

// Reads what the page cache holds of [off, off + bytes) without blocking on
// storage; returns the bytes read (0 when nothing is cached or the file system
// refuses RWF_NOWAIT) or -errno.
int64_t read_cached(sh_file* f, uint8_t* dst, uint64_t off, uint64_t bytes) {
  if (f->nowait_refused.load(std::memory_order_relaxed)) return 0;
  uint64_t done = 0;
  while (done < bytes) {
    struct iovec iov;
    iov.iov_base = dst + done;
    iov.iov_len = (size_t)std::min<uint64_t>(bytes - done, 1ull << 30);
    const ssize_t r = ::preadv2(f->fd, &iov, 1, (off_t)(off + done), RWF_NOWAIT);
    f->reads.fetch_add(1, std::memory_order_relaxed);
    if (r > 0) {
      done += (uint64_t)r;
      continue;
    }
    if (r == 0) return -ENODATA;
    if (errno == EINTR) continue;
    if (errno == EAGAIN) break;
    if (errno == EOPNOTSUPP || errno == EINVAL || errno == ENOSYS) {
      f->nowait_refused.store(true, std::memory_order_relaxed);
      break;
    }
    return -errno;
  }
  f->bytes_cached.fetch_add(done, std::memory_order_relaxed);
  return (int64_t)done;
}

constexpr size_t kColdStreams = 4;

// The descriptor of cold-read stream k of f (its own open file, so its own
// read-ahead state); fd itself when another cannot be opened.
int stream_fd(sh_file* f, size_t k) {
  if (k == 0) return f->fd;
  std::lock_guard<std::mutex> g(f->stream_mu);
  if (f->stream_fd[k] < 0) f->stream_fd[k] = ::open(f->path.c_str(), O_RDONLY | O_CLOEXEC);
  return f->stream_fd[k] >= 0 ? f->stream_fd[k] : f->fd;
}

int read_buffered(sh_file* f, uint8_t* dst, uint64_t off, uint64_t bytes) {
  const int e = pread_full(f, f->fd, dst, off, bytes);
  if (e == 0) f->bytes_buffered.fetch_add(bytes, std::memory_order_relaxed);
  return e;
}

// Per-thread bounce buffer for direct reads into memory that cannot take a DMA (one piece
// plus alignment slack). It hangs off a pthread key whose destructor is libc's free, so a
// thread's buffer is freed when the thread ends and the library registers no thread-exit
// handler of its own (a C++ thread_local with a destructor would).
pthread_key_t g_bounce_key;
pthread_once_t g_bounce_once = PTHREAD_ONCE_INIT;
bool g_bounce_key_ok = false;

uint8_t* bounce_buffer() {
  (void)pthread_once(&g_bounce_once, [] { g_bounce_key_ok = pthread_key_create(&g_bounce_key, free) == 0; });
  if (!g_bounce_key_ok) return nullptr;
  void* p = pthread_getspecific(g_bounce_key);
  if (p == nullptr) {
    if (posix_memalign(&p, kAlign, kPiece + 2 * kAlign) != 0) return nullptr;
    if (pthread_setspecific(g_bounce_key, p) != 0) {
      free(p);
      return nullptr;
    }
  }
  return static_cast<uint8_t*>(p);
}

constexpr uint64_t align_down(uint64_t x) { return x & ~(kAlign - 1); }
constexpr uint64_t align_up(uint64_t x) { return (x + kAlign - 1) & ~(kAlign - 1); }

// Direct read of [off, off + bytes) through the bounce buffer. Returns 0, an
// errno, or EINVAL when the file system refuses the direct read.
int read_bounced(sh_file* f, int dfd, uint8_t* dst, uint64_t off, uint64_t bytes) {
  uint8_t* bb = bounce_buffer();
  if (bb == nullptr) return ENOMEM;
  while (bytes > 0) {
    const uint64_t a = align_down(off);
    const uint64_t lim = std::min<uint64_t>(a + kPiece, align_up(off + bytes));
    uint64_t got = 0;
    while (a + got < lim) {
      const ssize_t r = ::pread(dfd, bb + got, (size_t)(lim - a - got), (off_t)(a + got));
      f->reads.fetch_add(1, std::memory_order_relaxed);
      if (r < 0 && errno == EINTR) continue;
      if (r < 0) return errno;
      if (r == 0) break;  // end of file inside the aligned cover
      got += (uint64_t)r;
      if (((uint64_t)r & (kAlign - 1)) != 0) break;
    }
    if (a + got <= off) return ENODATA;
    const uint64_t n = std::min<uint64_t>(a + got, off + bytes) - off;
    std::memcpy(dst, bb + (off - a), n);
    f->bytes_bounced.fetch_add(n, std::memory_order_relaxed);
    dst += n;
    off += n;
    bytes -= n;
  }
  return 0;
}

// Zero-copy direct read of the aligned middle of a congruent piece; the head,
// the tail and whatever a short read leaves go through the page cache.
// Returns 0, an errno, or EFAULT / EINVAL before any byte was read.
int read_dma(sh_file* f, int dfd, uint8_t* dst, uint64_t off, uint64_t bytes) {
  const uint64_t a = align_up(off), b = align_down(off + bytes);
  uint64_t done = 0;  // bytes of [a, b) read with O_DIRECT
  while (a + done < b) {
    const size_t want = (size_t)std::min<uint64_t>(b - a - done, 1ull << 30);
    const ssize_t r = ::pread(dfd, dst + (a - off) + done, want, (off_t)(a + done));
    f->reads.fetch_add(1, std::memory_order_relaxed);
    if (r < 0 && errno == EINTR) continue;
    if (r < 0 && done == 0 && (errno == EFAULT || errno == EINVAL)) return errno;
    if (r < 0) return errno;
    if (r == 0) return ENODATA;
    done += (uint64_t)r;
    if (((uint64_t)r & (kAlign - 1)) != 0) break;  // short and unaligned: finish buffered
  }
  f->bytes_direct.fetch_add(done, std::memory_order_relaxed);
  int e = 0;
  if (a > off) e = read_buffered(f, dst, off, a - off);
  if (e == 0 && a + done < off + bytes) e = read_buffered(f, dst + (a + done - off), a + done, off + bytes - a - done);
  return e;
}

// Reads one piece (see the file comment for the routes).
int read_piece(sh_file* f, uint8_t* dst, uint64_t off, uint64_t bytes) {
  const int dfd = f->dfd.load(std::memory_order_relaxed);
  if (dfd < 0) return read_buffered(f, dst, off, bytes);
  if (!f->dma_refused.load(std::memory_order_relaxed) && (((uintptr_t)dst ^ off) & (kAlign - 1)) == 0 &&
      align_down(off + bytes) > align_up(off)) {
    const int e = read_dma(f, dfd, dst, off, bytes);
    if (e != EFAULT && e != EINVAL) return e;
    if (e == EFAULT) f->dma_refused.store(true, std::memory_order_relaxed);
  }
  const int e = read_bounced(f, dfd, dst, off, bytes);
  if (e != EINVAL) return e;
  // the file system wants a larger alignment or no direct I/O at all
  f->dfd.store(-1, std::memory_order_relaxed);
  return read_buffered(f, dst, off, bytes);
}

}  // namespace

// ── internal helpers shared with the loader ─────────────────────────────

void sh::append_copy(std::vector<IoPiece>& out, void* dst, const void* src, uint64_t bytes) {
  for (uint64_t o = 0; o < bytes; o += kPiece) {
    IoPiece p;
    p.dst = (uint8_t*)dst + o;
    p.src = (const uint8_t*)src + o;
    p.file = nullptr;
    p.file_off = 0;
    p.bytes = std::min<uint64_t>(kPiece, bytes - o);
    out.push_back(p);
  }
}

void sh::append_read(std::vector<IoPiece>& out, sh_file* f, uint64_t file_off, uint64_t bytes, void* dst) {
  uint64_t o = 0;
  while (o < bytes) {
    const uint64_t pos = file_off + o;
    const uint64_t next = std::min<uint64_t>((pos / kPiece + 1) * kPiece, file_off + bytes);
    IoPiece p;
    p.dst = (uint8_t*)dst + o;
    p.src = nullptr;
    p.file = f;
    p.file_off = pos;
    p.bytes = next - pos;
    out.push_back(p);
    o += p.bytes;
  }
}

int sh::check_range(const sh_file* f, uint64_t file_off, uint64_t bytes, const char* who) {
  if (f == nullptr) return sh::fail(SH_ERR_INVALID, "%s: file is NULL", who);
  if (file_off > f->size || bytes > f->size - file_off)
    return sh::fail(SH_ERR_INVALID, "%s: range [%llu, +%llu) is past the end of %s (%llu bytes)", who,
                    (unsigned long long)file_off, (unsigned long long)bytes, f->path.c_str(),
                    (unsigned long long)f->size);
  return SH_OK;
}

int sh::run_io(const std::vector<IoPiece>& pieces, int threads) {
  std::mutex mu;
  int first_errno = 0;
  const IoPiece* failed = nullptr;
  auto fail_at = [&](const IoPiece* p, int e) {
    std::lock_guard<std::mutex> g(mu);
    if (failed == nullptr) {
      failed = p;
      first_errno = e;
    }
  };
  // phase 1, every thread: copies, direct reads, and what the page cache holds
  std::vector<uint64_t> hot(pieces.size(), 0);
  sh::parallel_for(pieces.size(), threads > 0 ? (unsigned)threads : 1u, [&](size_t i) {
    const IoPiece& p = pieces[i];
    if (p.file == nullptr) {
      std::memcpy(p.dst, p.src, p.bytes);
      hot[i] = p.bytes;
      return;
    }
    if (p.file->dfd.load(std::memory_order_relaxed) >= 0 || p.file->nowait_refused.load(std::memory_order_relaxed)) {
      // direct reads run in parallel; without RWF_NOWAIT a piece may be cached: read it here
      const int e = read_piece(p.file, p.dst, p.file_off, p.bytes);
      if (e != 0) fail_at(&p, e);
      hot[i] = p.bytes;
      return;
    }
    const int64_t h = read_cached(p.file, p.dst, p.file_off, p.bytes);
    if (h < 0) {
      fail_at(&p, (int)-h);
      hot[i] = p.bytes;
      return;
    }
    hot[i] = (uint64_t)h;
    if ((uint64_t)h == p.bytes) p.file->bytes_buffered.fetch_add(p.bytes, std::memory_order_relaxed);
  });
  // phase 2: the cold remainders in file order, cut into contiguous runs of
  // about equal size, each read front to back by one thread on its own descriptor
  if (failed == nullptr) {
    std::vector<size_t> cold;
    uint64_t cold_bytes = 0;
    for (size_t i = 0; i < pieces.size(); ++i)
      if (hot[i] < pieces[i].bytes) {
        cold.push_back(i);
        cold_bytes += pieces[i].bytes - hot[i];
      }
    std::sort(cold.begin(), cold.end(), [&](size_t a, size_t b) {
      const IoPiece &x = pieces[a], &y = pieces[b];
      return x.file != y.file ? x.file < y.file : x.file_off < y.file_off;
    });
    const size_t n_runs = std::min<size_t>(kColdStreams, cold.size());
    std::vector<size_t> run_begin(n_runs + 1, cold.size());
    if (n_runs > 0) {
      run_begin[0] = 0;
      uint64_t acc = 0;
      size_t r = 1;
      for (size_t j = 0; j < cold.size() && r < n_runs; ++j) {
        acc += pieces[cold[j]].bytes - hot[cold[j]];
        if (acc * n_runs >= cold_bytes * r) run_begin[r++] = j + 1;
      }
    }
    sh::parallel_for(n_runs, (unsigned)n_runs, [&](size_t r) {
      for (size_t j = run_begin[r]; j < run_begin[r + 1]; ++j) {
        const IoPiece& p = pieces[cold[j]];
        const uint64_t h = hot[cold[j]];
        const int e = pread_full(p.file, stream_fd(p.file, r), p.dst + h, p.file_off + h, p.bytes - h);
        if (e != 0) {
          fail_at(&p, e);
          return;
        }
        p.file->bytes_buffered.fetch_add(p.bytes, std::memory_order_relaxed);
      }
    });
  }
  if (failed != nullptr)
    return sh::fail(SH_ERR_IO, "read of %llu bytes at offset %llu of %s failed: %s",
                    (unsigned long long)failed->bytes, (unsigned long long)failed->file_off,
                    failed->file->path.c_str(), first_errno == ENODATA ? "unexpected end of file" : strerror(first_errno));
  return SH_OK;
}

int sh::advice_fd(const sh_file* f) {
  return (f != nullptr && f->dfd.load(std::memory_order_relaxed) < 0) ? f->fd : -1;
}

// ── C ABI ───────────────────────────────────────────────────────────────

extern "C" int sh_file_open(const char* path, int flags, sh_file** out) {
  sh::clear_error();
  if (path == nullptr || out == nullptr) return sh::fail(SH_ERR_INVALID, "sh_file_open: NULL argument");
  if (flags & ~SH_FILE_DIRECT) return sh::fail(SH_ERR_INVALID, "sh_file_open: unknown flags %#x", flags);
  *out = nullptr;
  const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return sh::fail(SH_ERR_IO, "sh_file_open: cannot open %s: %s", path, strerror(errno));
  struct stat st;
  if (::fstat(fd, &st) != 0) {
    const int e = errno;
    ::close(fd);
    return sh::fail(SH_ERR_IO, "sh_file_open: cannot stat %s: %s", path, strerror(e));
  }
  if (!S_ISREG(st.st_mode)) {
    ::close(fd);
    return sh::fail(SH_ERR_INVALID, "sh_file_open: %s is not a regular file", path);
  }
  sh_file* f = new (std::nothrow) sh_file();
  if (f == nullptr) {
    ::close(fd);
    return sh::fail(SH_ERR_OOM, "sh_file_open: out of host memory");
  }
  f->fd = fd;
  f->size = (uint64_t)st.st_size;
  f->path = path;
  if (flags & SH_FILE_DIRECT) {
    const int dfd = ::open(path, O_RDONLY | O_CLOEXEC | O_DIRECT);
    f->dfd_owned = dfd;  // -1 when the file system refuses O_DIRECT: buffered reads only
    f->dfd.store(dfd);
  }
  *out = f;
  return SH_OK;
}

extern "C" int sh_file_close(sh_file* f) {
  sh::clear_error();
  if (f == nullptr) return SH_OK;
  if (f->dfd_owned >= 0) ::close(f->dfd_owned);
  for (int sfd : f->stream_fd)
    if (sfd >= 0) ::close(sfd);
  ::close(f->fd);
  delete f;
  return SH_OK;
}

extern "C" int sh_file_get_info(sh_file* f, sh_file_info* info) {
  sh::clear_error();
  if (f == nullptr || info == nullptr) return sh::fail(SH_ERR_INVALID, "sh_file_get_info: NULL argument");
  info->size = f->size;
  info->direct = f->dfd.load() >= 0 ? 1 : 0;
  info->bytes_direct = f->bytes_direct.load();
  info->bytes_bounced = f->bytes_bounced.load();
  info->bytes_buffered = f->bytes_buffered.load();
  info->bytes_cached = f->bytes_cached.load();
  info->reads = f->reads.load();
  return SH_OK;
}

extern "C" int sh_file_advise(sh_file* f, uint64_t offset, uint64_t bytes, int advice) {
  sh::clear_error();
  if (f == nullptr) return sh::fail(SH_ERR_INVALID, "sh_file_advise: file is NULL");
  int a = 0;
  if (advice == SH_FILE_WILLNEED) a = POSIX_FADV_WILLNEED;
  else if (advice == SH_FILE_DONTNEED) a = POSIX_FADV_DONTNEED;
  else return sh::fail(SH_ERR_INVALID, "sh_file_advise: unknown advice %d", advice);
  const int e = ::posix_fadvise(f->fd, (off_t)offset, (off_t)bytes, a);
  if (e != 0) return sh::fail(SH_ERR_IO, "sh_file_advise: posix_fadvise on %s: %s", f->path.c_str(), strerror(e));
  return SH_OK;
}

extern "C" int sh_file_read_batch(const sh_file_range* ranges, size_t n, void* base, int threads) {
  sh::clear_error();
  if (n > 0 && (ranges == nullptr || base == nullptr)) return sh::fail(SH_ERR_INVALID, "sh_file_read_batch: NULL argument");
  std::vector<sh::IoPiece> pieces;
  for (size_t i = 0; i < n; ++i) {
    const sh_file_range& r = ranges[i];
    if (int st = sh::check_range(r.file, r.file_off, r.bytes, "sh_file_read_batch")) return st;
    sh::append_read(pieces, r.file, r.file_off, r.bytes, (uint8_t*)base + r.dst);
  }
  return sh::run_io(pieces, threads);
}
