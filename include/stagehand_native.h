/*
 * stagehand_native.h — C ABI of the MI355X weight-streaming data path.
 *
 * Every entry point returns an int status (SH_OK on success). On failure the
 * calling thread's last-error string (sh_last_error) names the call and the
 * cause. No torch types cross this boundary: device buffers are raw device
 * pointers owned by the caller (PyTorch tensors in the Python layer), streams
 * and events are opaque handles (hipStream_t / hipEvent_t values; a torch
 * stream's `cuda_stream` integer may be passed as a stream handle).
 *
 * Status → Python exception mapping used by the binding (stagehand_amd/_native.py):
 *   SH_ERR_INVALID   → ValueError          (reference: PyValueError, turbo_src/lib.rs:59-61;
 *                                           VmmError::InvalidSlab/InvalidRegion, vmm_src/error.rs:30-53)
 *   SH_ERR_HIP       → RuntimeError        (reference: "CUDA error {code}", turbo_src/cuda_ffi.rs:62-69)
 *   SH_ERR_OOM       → StagehandOOMError   (reference: pool capacity, src/stagehand/pool.py:133-139)
 *   SH_ERR_WATERMARK → MemoryError         (reference: VmmError::Watermarked/NoEvictableRegions)
 *   SH_ERR_STATE     → RuntimeError        (reference: "No free GPU slots", turbo_src/engine.rs:189)
 *   SH_ERR_NOT_READY → not an error: the queried event/transfer is still pending
 *   SH_ERR_TIMEOUT   → TimeoutError
 *   SH_ERR_IO        → OSError             (reference: open/mmap of a weight file, src/stagehand/scheduler.py:564-601)
 */
#ifndef STAGEHAND_NATIVE_H
#define STAGEHAND_NATIVE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SH_ABI_VERSION 8

enum sh_status {
  SH_OK = 0,
  SH_ERR_INVALID = 1,
  SH_ERR_HIP = 2,
  SH_ERR_OOM = 3,
  SH_ERR_NOT_READY = 4,
  SH_ERR_STATE = 5,
  SH_ERR_TIMEOUT = 6,
  SH_ERR_WATERMARK = 7,
  SH_ERR_IO = 8
};

/* Thread-local description of the last failure on the calling thread. */
const char* sh_last_error(void);
/* SH_ABI_VERSION of the loaded library. */
int sh_abi_version(void);

/* Process teardown. The reference's native engines release their threads, streams and
 * pinned memory in their Rust Drop impls when Python drops them (turbo_src/engine.rs:395-422,
 * vmm_src/allocator.rs:648-713, the prefetch thread's join in vmm_src/prefetch.rs:22-46).
 * Here each object's destroy call does that, and sh_shutdown ends what the library holds
 * for the whole process: it joins the shared host copy threads (at once, or when a copy
 * still running on another thread returns; they start again on the next use), and, when no
 * loader, save-back or turbo engine is alive, waits for each device that ran the library's
 * kernels and unloads their code (loaded again on the next use). The library registers no
 * exit-time handler of its own: a process that never calls sh_shutdown leaves the loaded code
 * to the HIP runtime's own teardown. No other call of the library may run while sh_shutdown
 * does (a launch racing the unload would use freed code). It fills `live` (may be NULL) with the
 * native objects not yet destroyed, so a caller at interpreter exit can check that nothing still
 * runs when the HIP runtime is torn down. */
typedef struct sh_live_counts {
  uint64_t pools, loaders, savebacks, turbos, vmms, files;
  uint64_t copy_threads;   /* host copy threads still running */
  uint64_t kernel_devices; /* devices on which the kernels' code is still loaded */
} sh_live_counts;
int sh_shutdown(sh_live_counts* live);

/* ───────────────────────── device, streams, events, copies ─────────────────────────
 * HIP rewrite of the CUDA runtime FFI the reference declares by hand in
 * turbo_src/cuda_ffi.rs:26-59 (cudaSetDevice, cudaStreamCreateWithFlags,
 * cudaEventCreateWithFlags/Record/Query/Synchronize, cudaStreamWaitEvent,
 * cudaMemcpyAsync, cudaMallocHost/cudaFreeHost). */

int sh_device_count(int* count);
int sh_set_device(int device);                     /* cudaSetDevice, turbo_src/cuda_ffi.rs:57 */
int sh_get_device(int* device);

/* Pinned host memory (hipHostMalloc, coherent default flags).
 * Replaces cudaMallocHost/cudaFreeHost, turbo_src/cuda_ffi.rs:29-30. */
int sh_host_alloc(size_t bytes, void** out);
int sh_host_free(void* ptr);

/* Non-blocking stream at the default priority.
 * Replaces cudaStreamCreateWithFlags(.., 1), turbo_src/cuda_ffi.rs:44 and the
 * torch.cuda.Stream of src/stagehand/transfer.py:95-98. */
int sh_stream_create(void** out);
int sh_stream_destroy(void* stream);
int sh_stream_sync(void* stream);                  /* cudaStreamSynchronize, turbo_src/cuda_ffi.rs:45 */
int sh_stream_wait_event(void* stream, void* event); /* cudaStreamWaitEvent, turbo_src/cuda_ffi.rs:54 */

/* timing != 0 creates a timing event (for sh_event_elapsed_ms); otherwise
 * hipEventDisableTiming as in turbo_src/cuda_ffi.rs:49 + EVENT_DISABLE_TIMING. */
int sh_event_create(int timing, void** out);
int sh_event_destroy(void* event);
int sh_event_record(void* event, void* stream);    /* cudaEventRecord, turbo_src/cuda_ffi.rs:50 */
int sh_event_query(void* event);                   /* SH_OK when complete, SH_ERR_NOT_READY when pending */
int sh_event_sync(void* event);                    /* cudaEventSynchronize, turbo_src/cuda_ffi.rs:51 */
int sh_event_elapsed_ms(void* start, void* end, float* ms);

/* Async copies on `stream` (cudaMemcpyAsync kinds 1/2, turbo_src/cuda_ffi.rs:35-41). */
int sh_memcpy_h2d_async(void* dst_dev, const void* src_host, size_t bytes, void* stream);
int sh_memcpy_d2h_async(void* dst_host, const void* src_dev, size_t bytes, void* stream);
int sh_memcpy_d2d_async(void* dst_dev, const void* src_dev, size_t bytes, void* stream);

/* ───────────────────────── slab unpack (dequant / cast) ─────────────────────────
 * A plan describes how one packed source slab (already in device memory) is
 * scattered into one destination buffer (a block's contiguous parameter
 * buffer laid out as in src/stagehand/scheduler.py:148-165: params in
 * named_parameters() order, offset = running sum of numel * itemsize, no padding).
 *
 * One descriptor per parameter region:
 *   SH_KIND_I8_ROWSCALE_BF16  dst[r*cols+c] = bf16_rne((f32(q[r*src_ld+c]) - zp[r]) * scale[r])
 *                             the SquareQ dequant of src/stagehand/scheduler.py:290-300
 *                             (q2d = qweight.reshape(rows,-1)[:out,:in]; src_ld = padded_in).
 *                             zp is optional (NULL zero_points ⇒ the subtraction is skipped,
 *                             which is bit-identical to subtracting 0.0f).
 *   SH_KIND_I8_ROWSCALE_F32   same, fp32 output (runtime dtype float32).
 *   SH_KIND_F32_BF16          dst[i] = bf16_rne(src_f32[i]); the fp32→bf16 casts of
 *                             src/stagehand/scheduler.py:181, 224-230, 305, 1071.
 *   SH_KIND_BF16_F32          dst[i] = f32(src_bf16[i]) (exact widening).
 *   SH_KIND_COPY_BYTES        dst[i] = src[i] for cols bytes (same-dtype sources: bf16→bf16).
 *   SH_KIND_ZERO_BYTES        dst[i] = 0 for cols bytes (the zero-fill fallbacks of
 *                             src/stagehand/scheduler.py:240, 276-297, 325).
 * bf16_rne is round-to-nearest-even of the fp32 bit pattern; every NaN maps to
 * 0xFFFF, which is what torch's CPU float→bfloat16 conversion produces.
 *
 * rows/cols/src_ld are in elements of the source kind (bytes for the *_BYTES
 * kinds, where rows must be 1). scale_off indexes `scales` / `zero_points`.
 * Fields after scale_off are filled in by sh_plan_create and ignored on input.
 */
enum sh_kind {
  SH_KIND_I8_ROWSCALE_BF16 = 1,
  SH_KIND_I8_ROWSCALE_F32 = 2,
  SH_KIND_F32_BF16 = 3,
  SH_KIND_BF16_F32 = 4,
  SH_KIND_COPY_BYTES = 5,
  SH_KIND_ZERO_BYTES = 6
};

typedef struct sh_unpack_desc {
  uint64_t src_off;    /* byte offset of source element (0,0) in the source buffer */
  uint64_t dst_off;    /* byte offset of destination element 0 in the destination buffer */
  uint32_t rows;       /* rows (output features); 1 for flat regions */
  uint32_t cols;       /* elements per row that are written */
  uint32_t src_ld;     /* source row stride in elements (>= cols); 0 means cols */
  uint32_t kind;       /* enum sh_kind */
  uint64_t scale_off;  /* index of row 0's scale / zero point */
  /* filled by sh_plan_create: */
  uint64_t div_magic;  /* ceil(2^64 / cols), 0 when cols == 1 */
  uint32_t tile_begin; /* first tile of this descriptor */
  uint32_t ntiles;     /* tiles covering rows*cols elements */
  uint32_t lead;       /* elements before element 0 in the first tile, so that the tiles' destination
                          spans start on 4 KiB boundaries (0 when the region start allows none) */
  uint32_t reserved;
} sh_unpack_desc;     /* 64 bytes, identical layout on host and device */

typedef struct sh_plan sh_plan;

typedef struct sh_plan_info {
  uint32_t n_desc;          /* descriptors after splitting oversize regions */
  uint32_t n_tiles;         /* workgroups per launch */
  uint32_t kind_mask;       /* bit (1 << kind) for every kind present */
  uint32_t tile_elems;      /* elements per tile */
  uint64_t src_extent;      /* bytes of source the plan reads (max src end) */
  uint64_t dst_extent;      /* bytes of destination the plan writes (max dst end) */
  uint64_t scale_extent;    /* scale / zero-point entries the plan reads */
  uint64_t algo_bytes;      /* algorithmic HBM bytes per launch (reads + writes) */
  uint64_t elements;        /* elements written */
} sh_plan_info;

/* Validates the descriptors, splits regions above 2^31 elements by rows, and
 * uploads the descriptor table and tile map to the current device (the only
 * device allocation of the unpack path; done once per block layout). */
int sh_plan_create(const sh_unpack_desc* descs, uint32_t n, sh_plan** out);
int sh_plan_destroy(sh_plan* plan);
/* Host-only validation of a descriptor table: fills `info` exactly as
 * sh_plan_create would, without touching a device. */
int sh_plan_describe(const sh_unpack_desc* descs, uint32_t n, sh_plan_info* info);
int sh_plan_get_info(const sh_plan* plan, sh_plan_info* info);

/* Generic launch: one kernel over every descriptor of the plan, on `stream`.
 * The byte/entry sizes of the buffers are checked against the plan's extents
 * before anything is launched. scales/zero_points may be NULL when the plan has
 * no I8 descriptor; zero_points may always be NULL. */
int sh_unpack(const sh_plan* plan,
              const void* src, size_t src_bytes,
              const float* scales, const float* zero_points, size_t n_scale,
              void* dst, size_t dst_bytes, void* stream);

/* SquareQ INT8→bf16 dequant. Replaces the host dequant of
 * src/stagehand/scheduler.py:243-325 (core expression :299-300). The plan must
 * hold only SH_KIND_I8_ROWSCALE_BF16 descriptors. */
int sh_dequant_i8_rowscale_bf16(const sh_plan* plan,
                                const int8_t* src, size_t src_bytes,
                                const float* scales, const float* zero_points, size_t n_scale,
                                uint16_t* dst, size_t dst_bytes, void* stream);

/* fp32→bf16 slab unpack/cast. Replaces the host casts of
 * src/stagehand/scheduler.py:168-181 and :1066-1071. The plan must hold only
 * SH_KIND_F32_BF16 descriptors. */
int sh_unpack_cast_f32_bf16(const sh_plan* plan,
                            const float* src, size_t src_bytes,
                            uint16_t* dst, size_t dst_bytes, void* stream);

/* No counterpart in the reference: for callers that cannot allocate device memory — code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc. It does what
 * sh_plan_create + sh_unpack + sh_plan_destroy do for `descs`, with the same kernels and the
 * same results, but the plan's launch table and tile map go into a static device array of
 * SH_UNPACK_NOALLOC_SCRATCH_BYTES (8 MiB) in the library's code object, one per GPU it runs on,
 * held until sh_shutdown unloads the kernels (or the process ends); it calls no device
 * allocator. Descriptors reach the device as kernel arguments, so nothing on the host has to
 * outlive the call. Limits: at most SH_UNPACK_NOALLOC_MAX_DESCS descriptors after the plan's
 * splitting of oversize regions and SH_UNPACK_NOALLOC_MAX_TILES tiles (config 2's dequant
 * needs 270k, its cast 1.08 M); beyond them it returns SH_ERR_INVALID. All calls on one GPU
 * share its array and leave the last call's table in it. Each call's kernels wait on the
 * device for the previous call's on that GPU (an event recorded after every call), so calls
 * from several streams or threads do not corrupt each other. A call made while `stream` is
 * being captured into a graph is not ordered that way (its kernels run at the graph's
 * replays): such replays must not overlap other calls on that GPU. The first call on a GPU
 * loads the kernels there (as every entry point's first launch does) and creates the event. */
#define SH_UNPACK_NOALLOC_MAX_DESCS 2048u
#define SH_UNPACK_NOALLOC_MAX_TILES 2064384u
#define SH_UNPACK_NOALLOC_SCRATCH_BYTES (8u << 20)
int sh_unpack_noalloc(const sh_unpack_desc* descs, uint32_t n,
                      const void* src, size_t src_bytes,
                      const float* scales, const float* zero_points, size_t n_scale,
                      void* dst, size_t dst_bytes, void* stream);

/* ───────────────────────── pinned slab pool ─────────────────────────
 * Replaces the torch pinned-tensor pool of src/stagehand/pool.py:42-246
 * (PinnedPool.__init__ :58-116, acquire :122-175, release :181-196,
 * stats :202-212, shutdown :218-226). One pinned region (hipHostMalloc) cut
 * into equal slabs; pinned == 0 gives ordinary aligned host memory (the
 * reference's no-GPU fallback, pool.py:87). */
typedef struct sh_pool sh_pool;
typedef struct sh_pool_stats {
  uint64_t total;        /* slabs */
  uint64_t free;         /* slabs on the free list */
  uint64_t in_use;       /* acquired or awaiting their release event */
  uint64_t peak_in_use;
  uint64_t wait_count;   /* acquires that had to wait */
  uint64_t fenced;       /* released slabs whose release event has not completed */
  double total_wait_ms;
  uint64_t slab_bytes;
  uint64_t pinned;
} sh_pool_stats;

int sh_pool_create(uint32_t num_slabs, uint64_t slab_bytes, int pinned, sh_pool** out);
int sh_pool_destroy(sh_pool* pool);
int sh_pool_slab_ptr(sh_pool* pool, uint32_t slab, void** ptr);
/* Blocks until a slab is free (timeout_ms < 0: no limit; SH_ERR_TIMEOUT when it
 * expires). waited_ms (may be NULL) receives the time spent waiting. */
int sh_pool_acquire(sh_pool* pool, int64_t timeout_ms, uint32_t* slab, double* waited_ms);
int sh_pool_release(sh_pool* pool, uint32_t slab);
/* No reference counterpart: the slab returns to the free list once all work
 * queued on `stream` so far has completed (an event the pool records), so the
 * host need not wait for an H2D copy before recycling its source slab. */
int sh_pool_release_after(sh_pool* pool, uint32_t slab, void* stream);
int sh_pool_get_stats(sh_pool* pool, sh_pool_stats* stats);

/* ───────────────────────── weight files ─────────────────────────
 * Bulk reads of weight files into host memory: the replacement of the
 * per-parameter reads through an mmap (torch.frombuffer over the mapping, then
 * copy_ into the slab) of src/stagehand/scheduler.py:184-241 and 564-601, and
 * of the VMM backend's mmap fills with madvise(WILLNEED) read-ahead
 * (src/stagehand/vmm_backend.py:283-291).
 *
 * A read is cut into pieces of at most 8 MiB at 8 MiB file offsets, spread
 * over the host copy threads, which first copy what the page cache holds
 * (preadv2 RWF_NOWAIT); the rest is then read from storage in file order by
 * up to 4 threads, each reading one contiguous run front to back on a
 * descriptor of its own (interleaved cold reads of one file defeat the
 * kernel's read-ahead). A file opened with
 * SH_FILE_DIRECT also holds an O_DIRECT descriptor and is read around the page
 * cache: straight into the destination (the storage DMA writes it) where the
 * destination is congruent to the file offset modulo SH_FILE_ALIGN and the
 * kernel can pin it (the unaligned head and tail then go through the page
 * cache), else through a per-thread aligned bounce buffer — the route of
 * hipHostMalloc'd memory, which the kernel refuses to pin for a DMA. Where the
 * file system refuses O_DIRECT, the file is read buffered only
 * (sh_file_info.direct = 0). Reads past the end of the file (as sized when it
 * was opened) are SH_ERR_INVALID; failed reads SH_ERR_IO. */
#define SH_FILE_DIRECT 1
#define SH_FILE_ALIGN 4096
enum sh_file_advice { SH_FILE_WILLNEED = 1, SH_FILE_DONTNEED = 2 };
typedef struct sh_file sh_file;
typedef struct sh_file_info {
  uint64_t size;
  uint64_t direct;          /* 1 when an O_DIRECT descriptor is open */
  uint64_t bytes_direct;    /* bytes read with O_DIRECT into the destination so far */
  uint64_t bytes_bounced;   /* bytes read with O_DIRECT through the bounce buffer so far */
  uint64_t bytes_buffered;  /* bytes read through the page cache so far */
  uint64_t bytes_cached;    /* of those, bytes the page cache already held */
  uint64_t reads;           /* pread calls so far */
} sh_file_info;
typedef struct sh_file_range {
  sh_file* file;
  uint64_t file_off;
  uint64_t bytes;
  uint64_t dst;  /* byte offset from the destination base */
} sh_file_range;
int sh_file_open(const char* path, int flags, sh_file** out);
int sh_file_close(sh_file* f);
int sh_file_get_info(sh_file* f, sh_file_info* info);
/* posix_fadvise over [offset, offset + bytes) (bytes 0: to the end of the file). */
int sh_file_advise(sh_file* f, uint64_t offset, uint64_t bytes, int advice);
/* Reads every range to base + range.dst on up to `threads` copy threads. */
int sh_file_read_batch(const sh_file_range* ranges, size_t n, void* base, int threads);

/* Multi-threaded host memcpy of a batch of (dst, src, bytes) items, used to
 * gather a block's parameters into its pinned slab (the per-parameter host
 * copy_ loops of src/stagehand/scheduler.py:168-181, 203-241, 263-325). */
typedef struct sh_copy_item {
  void* dst;
  const void* src;
  uint64_t bytes;
} sh_copy_item;
int sh_host_copy_batch(const sh_copy_item* items, size_t n, int threads);

/* ───────────────────────── block loader ─────────────────────────
 * A native worker thread that performs a block load end to end: gather the
 * block's parameter bytes into a pinned slab (multi-threaded host copy), H2D
 * the slab on the loader's copy stream, and, with a plan, unpack it into the
 * destination. The unpack and the chunk digests (post-copy work) are queued by
 * the first call that needs them: sh_loader_stream_wait queues them on its
 * stream behind a device wait on the copy; sh_loader_query (once the copy has
 * landed), sh_loader_sync, sh_loader_release, sh_loader_ticket_times and
 * sh_loader_destroy queue them on the loader's unpack stream after the copy
 * has landed. No loader stream waits on the device for a copy still queued:
 * HIP runs the streams that share a hardware queue in the order their work was
 * queued, so such a wait could hold back the compute stream. Replaces the synchronous host
 * staging + copy + host wait of src/stagehand/scheduler.py:953-1031,
 * src/stagehand/transfer.py:108-143 / 193-217 and the prefetch half of
 * turbo_src/engine.rs:202-282.
 *
 * pieces[i].dst is a BYTE OFFSET inside the slab (not a pointer); src is a
 * host pointer that must stay valid until the ticket is issued (sh_loader_query
 * no longer returns SH_ERR_NOT_READY for the staging phase, i.e. after
 * sh_loader_stream_wait / sh_loader_sync / a successful query).
 * The source streams through the pool in slab-sized chunks (a block may be
 * larger than one slab; the reference requires it to fit one, pool.py:133-175
 * with scheduler.py:970). Without a plan the src_bytes are copied to dst; with
 * a plan they are copied to `staging` (device) and unpacked into dst, with the
 * fp32 scales / zero points read from staging + scale_off / zp_off
 * (zp_off < 0: no zero points). The copy waits for the work queued on
 * `wait_stream` at submit time (the destination's allocation stream). */
typedef struct sh_load_request {
  const sh_copy_item* pieces;
  uint64_t n_pieces;
  uint64_t src_bytes;
  const sh_plan* plan;
  void* staging;
  uint64_t staging_bytes;
  void* dst;
  uint64_t dst_bytes;
  int64_t scale_off;
  int64_t zp_off;
  uint64_t n_scale;
  int32_t copy_threads;  /* host copy threads for this request; <= 0: loader default */
  int32_t reserved;
  /* Optional pinned host image of the whole source (src_bytes; from
   * sh_host_alloc). When set, the pieces are gathered into the image (offsets
   * relative to it; n_pieces may be 0 when it already holds them) and the H2D
   * reads the image directly, with no pool slab — the turbo engine's
   * all-blocks-pinned layout (turbo_src/engine.rs:132-138) for sources that do
   * not change. Before re-gathering into an image the loader waits for the
   * previous copy out of it. */
  void* image;
  /* Optional file ranges (sh_file_range, dst = byte offset in the source like
   * pieces[i].dst), read into the slab chunks (or the image) by the same copy
   * threads, with pread / O_DIRECT (sh_file_open). The files must stay open
   * until the ticket is issued. When the loader starts a ticket, it asks the
   * kernel to read ahead (POSIX_FADV_WILLNEED) the buffered ranges of that
   * ticket and of the ticket queued after it. */
  const struct sh_file_range* ranges;
  uint64_t n_ranges;
  /* Optional pieces whose sources are pinned host memory (dst = byte offset
   * in the source, as for pieces): copied straight from their source to the
   * device by the copy engine, with no slab and no host copy. Their sources
   * are read until the load completes (not only until the ticket is issued,
   * as for pieces): keep them alive and unchanged until then. The regions of
   * the other pieces and ranges must not overlap them. */
  const sh_copy_item* dma;
  uint64_t n_dma;
  /* Optional event (hipEvent_t) the copies wait for on the device, e.g. the
   * device-to-host copy that wrote the pinned sources of `dma` (no reference
   * counterpart: the reference waits on the host before reading them again).
   * With a pinned image, the loader's worker waits for it on the host before
   * copying the dma pieces into the image. It must stay valid until the
   * ticket is issued. */
  void* wait_event;
  /* Optional save-back ticket (sh_saveback_submit) the loader's worker waits
   * for on the host before it issues any copy of this request, e.g. the SDMA
   * copy that wrote the pinned sources of `dma` (no reference counterpart, as
   * for wait_event). Do not release the ticket before the load completes. */
  struct sh_saveback* saveback;
  uint64_t saveback_ticket;
  /* Optional digests of the destination once written (no reference counterpart; for
   * sh_saveback_submit_chunks): sh_block_digest of dst[0, digest_bytes) in chunks of
   * digest_chunk bytes into `digest` (device memory), as post-copy work, before the load
   * counts as done. */
  uint64_t* digest;
  uint64_t digest_bytes;
  uint32_t digest_chunk;
  uint32_t reserved2;
} sh_load_request;

typedef struct sh_loader sh_loader;
int sh_loader_create(sh_pool* pool, int copy_threads, sh_loader** out);
int sh_loader_destroy(sh_loader* loader);
int sh_loader_streams(sh_loader* loader, void** copy_stream, void** unpack_stream);
int sh_loader_submit(sh_loader* loader, const sh_load_request* req, void* wait_stream, uint64_t* ticket);
/* SH_OK once the destination is written, SH_ERR_NOT_READY before. Queues the
 * post-copy work on the unpack stream once the copy has landed. */
int sh_loader_query(sh_loader* loader, uint64_t ticket);
/* Makes `stream` wait for the load on the device (the host waits only until
 * the worker has issued it). The first call for a ticket with post-copy work
 * queues that work on `stream`, behind a device wait on the copy. */
int sh_loader_stream_wait(sh_loader* loader, uint64_t ticket, void* stream);
/* Host waits until the destination is written. */
int sh_loader_sync(sh_loader* loader, uint64_t ticket);
/* The copy alone (no reference counterpart; the reference's transfer is its
 * copy, src/stagehand/transfer.py:126-143, which the in-flight bound of
 * transfer.py:258-276 counts): SH_OK once the ticket's host-to-device copies
 * have landed, whether or not its post-copy work has run, SH_ERR_NOT_READY
 * before; and a host wait for that point. The post-copy work of a ticket that
 * sh_loader_stream_wait queued on a compute stream completes only when that
 * stream reaches it, so a bound on copies in flight waits on these. */
int sh_loader_query_copy(sh_loader* loader, uint64_t ticket);
int sh_loader_sync_copy(sh_loader* loader, uint64_t ticket);
/* Forgets a ticket (waits for its device work first, post-copy work included:
 * the destination and digests are written on return). */
int sh_loader_release(sh_loader* loader, uint64_t ticket);
/* Timing of later submissions (no reference counterpart; the per-block copy
 * and unpack GB/s telemetry): when enabled, each ticket's copy-start,
 * copy-end and done points are timing events. sh_loader_ticket_times waits for
 * the ticket and returns the three times in ms after `ref_event` (a timing
 * event recorded earlier); call it before sh_loader_release. */
int sh_loader_set_timing(sh_loader* loader, int enable);
int sh_loader_ticket_times(sh_loader* loader, uint64_t ticket, void* ref_event, float* out3);

/* ───────────────────────── save-back copies on an SDMA engine ─────────────────────────
 * Device-to-host copies of evicted blocks' bytes into pinned host memory (the
 * reference copies back synchronously with `param.data.to("cpu")`,
 * src/stagehand/scheduler.py:1216-1226 and 1348-1366), issued on a system DMA
 * engine through the HSA runtime instead of hipMemcpyAsync, which runs a pinned
 * device-to-host copy as a kernel on the compute units and slows the compute
 * kernels beside it. A submit records an event on `stream`; the engine's worker
 * thread waits for it on the host and then issues the copies, so they read what
 * the work queued on `stream` before the submit wrote. items[i] is a (pinned
 * host dst, device src, bytes) triple; both buffers stay in use until the ticket
 * completes. Tickets complete in submission order: query and wait report a
 * ticket complete only when every earlier ticket not yet released is, so a later
 * ticket covers the copies of earlier ones. Consumers wait on the host (query,
 * wait) or in the loader (sh_load_request.saveback). No reference counterpart. */
typedef struct sh_saveback sh_saveback;
int sh_saveback_create(int device, sh_saveback** out);
/* Issues what is still queued, waits for every ticket, stops the worker and
 * frees the engine; returns the first copy failure, if any. */
int sh_saveback_destroy(sh_saveback* sb);
int sh_saveback_submit(sh_saveback* sb, const sh_copy_item* items, uint64_t n, void* stream, uint64_t* ticket);
/* As sh_saveback_submit, but the copies start once each of the n_events events
 * (hipEvent_t) has completed, instead of after everything queued on a stream:
 * the worker waits for each event on the host. The caller vouches that no work
 * queued after those events writes the sources, and keeps the events alive, and
 * does not record them again, until the ticket completes. An event recorded in
 * the middle of a busy compute stream completes there: no stream is needed, so
 * no hardware queue that the stream would share with that compute. No
 * reference counterpart. */
int sh_saveback_submit_after(sh_saveback* sb, const sh_copy_item* items, uint64_t n, void* const* events,
                             uint32_t n_events, uint64_t* ticket);
/* SH_OK when the ticket (and every earlier one) is complete, SH_ERR_NOT_READY
 * before, or the failure of a copy. */
int sh_saveback_query(sh_saveback* sb, uint64_t ticket);
int sh_saveback_wait(sh_saveback* sb, uint64_t ticket);
/* Waits for the ticket's own copies, then forgets it (releasing twice is a no-op). */
int sh_saveback_release(sh_saveback* sb, uint64_t ticket);
/* Timing (telemetry): with timing on, sh_saveback_ticket_times waits for a later
 * ticket and returns the start and end of its copies in ns of the HSA system
 * clock, which sh_saveback_clock_ns reads (for a ticket of several copies the
 * start is the issue of the first). Call it before releasing the ticket. */
int sh_saveback_set_timing(sh_saveback* sb, int enable);
int sh_saveback_clock_ns(uint64_t* ns);
int sh_saveback_ticket_times(sh_saveback* sb, uint64_t ticket, uint64_t* out2);
/* Save-back of the chunks that changed (no reference counterpart: the reference copies the
 * whole block back, src/stagehand/scheduler.py:1216-1226). Each region copies dev_src[0, bytes)
 * into host_dst (pinned) in chunks of chunk_bytes, only the chunks whose digest differs from
 * digests[2 * (first_chunk + c)], [.. + 1] (as sh_block_digest wrote them for that region,
 * device memory). The submit queues sh_block_changed for every region on `digest_stream`, after
 * the caller's events (or, with n_events == 0, after the work queued on `stream` now), into
 * changed[first_chunk + c] (pinned host memory, one byte per chunk); once that has run, the
 * engine's worker issues one copy per run of changed chunks. digests == NULL copies every chunk
 * (ordered as sh_saveback_submit / _submit_after). The caller vouches that each host_dst held the
 * bytes its digests describe. All buffers stay in use until the ticket completes;
 * sh_saveback_ticket_bytes then gives the bytes copied. */
typedef struct sh_chunk_region {
  void* host_dst;
  const void* dev_src;
  uint64_t bytes;
  uint64_t first_chunk; /* the region's first chunk in digests / changed */
} sh_chunk_region;
int sh_saveback_submit_chunks(sh_saveback* sb, const sh_chunk_region* regions, uint32_t n_regions, uint32_t chunk_bytes,
                              const uint64_t* digests, uint8_t* changed, void* digest_stream, void* const* events,
                              uint32_t n_events, void* stream, uint64_t* ticket);
/* Waits for the ticket and gives the bytes its copies moved. */
int sh_saveback_ticket_bytes(sh_saveback* sb, uint64_t ticket, uint64_t* bytes);

/* ───────────────────────── chunk digests ─────────────────────────
 * Per-chunk digests of a buffer (no reference counterpart), for sh_saveback_submit_chunks
 * and the load request's `digest`: two uint64 per chunk of chunk_bytes (a positive multiple
 * of 16; the last chunk may be shorter), the sums over the chunk's 8-byte words of two
 * bijective 64-bit mixes keyed by the word's position. A change of one word always changes a
 * chunk's digest. sh_block_digest writes digests[2c], digests[2c + 1] on `stream`;
 * sh_block_changed writes changed[c] = 1 where the chunk's digest differs from those, else 0;
 * sh_block_digest_host computes the same digests on the host. */
int sh_block_digest(const void* buf, uint64_t bytes, uint32_t chunk_bytes, uint64_t* digests, void* stream);
int sh_block_changed(const void* buf, uint64_t bytes, uint32_t chunk_bytes, const uint64_t* digests, uint8_t* changed,
                     void* stream);
int sh_block_digest_host(const void* buf, uint64_t bytes, uint32_t chunk_bytes, uint64_t* digests);

/* ───────────────────────── turbo window engine ─────────────────────────
 * A fixed window of device slots that blocks rotate through: the HIP rewrite
 * of the reference's Rust TransferEngine (turbo_src/engine.rs:51-422, Python
 * surface turbo_src/lib.rs:14-126). Every block's parameters live in ONE
 * pinned host region (params at 256-byte aligned offsets), so a block moves in
 * one hipMemcpyAsync when its slot is a contiguous device buffer
 * (sh_turbo_set_slot_buffer). The compute stream waits on the block's own H2D
 * event (no host synchronisation, no shared event), an eviction orders its
 * write-back after the compute queued so far, and a slot freed by an eviction
 * is reused by a prefetch through a device wait on the slot's fence; a
 * write-back on the SDMA engine (sh_turbo_set_save_back) is waited for on the
 * host by the prefetch that reuses its slot or reloads its block. Blocks marked
 * write-back off (frozen weights) skip the D2H and keep every wait on the
 * device. Device pointers in slots belong to the caller (PyTorch tensors),
 * pinned host memory to the engine (engine.rs:132-138, 396-422).
 * Errors: a bad direction is SH_ERR_INVALID (ValueError, lib.rs:59-61); every
 * other failure, including "No free GPU slots" (engine.rs:189) and an index
 * out of range, is SH_ERR_STATE or SH_ERR_HIP (RuntimeError, lib.rs:38-40). */
enum sh_turbo_location { SH_TURBO_CPU = 0, SH_TURBO_GPU = 1, SH_TURBO_H2D = 2, SH_TURBO_D2H = 3 };
enum sh_turbo_direction { SH_TURBO_FORWARD = 0, SH_TURBO_BACKWARD = 1 };
typedef struct sh_turbo sh_turbo;
int sh_turbo_create(sh_turbo** out);                                      /* TransferEngine::new, engine.rs:67-79 */
int sh_turbo_destroy(sh_turbo* t);                                        /* Drop, engine.rs:396-422 */
int sh_turbo_register_block(sh_turbo* t, const uint64_t* sizes, uint32_t n, uint32_t* index); /* engine.rs:82-99 */
int sh_turbo_initialize(sh_turbo* t, int device, uint32_t window);        /* engine.rs:102-156 */
int sh_turbo_stage_block(sh_turbo* t, uint32_t block, const void* const* src, uint32_t n); /* engine.rs:159-175 */
int sh_turbo_step(sh_turbo* t, uint32_t block, int direction, void* compute_stream);     /* engine.rs:304-341 */
int sh_turbo_evict_sync(sh_turbo* t, uint32_t block, void* compute_stream);             /* lib.rs:68-73 */
int sh_turbo_drain(sh_turbo* t);                                          /* lib.rs:108-118 */
int sh_turbo_gpu_ptr(sh_turbo* t, uint32_t block, uint32_t param, uint64_t* ptr);       /* engine.rs:344-350 */
int sh_turbo_cpu_ptr(sh_turbo* t, uint32_t block, uint32_t param, uint64_t* ptr);       /* engine.rs:353-358 */
int sh_turbo_set_slot_gpu_ptrs(sh_turbo* t, uint32_t slot, const uint64_t* ptrs, uint32_t n); /* engine.rs:361-372 */
/* No reference counterpart: a slot as one contiguous device buffer of at
 * least sh_turbo_slot_bytes bytes; a block's param p then sits at its own
 * aligned offset and the whole block is a single copy. */
int sh_turbo_set_slot_buffer(sh_turbo* t, uint32_t slot, void* base, uint64_t bytes);
int sh_turbo_slot_bytes(sh_turbo* t, uint64_t* bytes);
int sh_turbo_param_offset(sh_turbo* t, uint32_t block, uint32_t param, uint64_t* offset);
/* No reference counterpart (the reference always copies back): 0 skips the
 * D2H at eviction for a block whose device copy is never written. */
int sh_turbo_set_writeback(sh_turbo* t, uint32_t block, int enable);
/* No reference counterpart: before sh_turbo_initialize, where write-backs run.
 * 1 (the default): on an SDMA engine (sh_saveback); a prefetch that reuses the
 * slot of a block being written back, or reloads that block, waits for the copy
 * on the host (sh_turbo_step's lookahead prefetch leaves that wait, and its
 * copy, to the next engine call, with the block already marked h2d). 0:
 * hipMemcpyAsync on the engine's evict stream (a kernel on the compute units),
 * ordered on the device only. */
int sh_turbo_set_save_back(sh_turbo* t, int sdma);
/* Before sh_turbo_initialize (no reference counterpart): write-backs on the SDMA engine copy
 * back only the chunks of chunk_bytes (a multiple of 16; default 256 KiB) that changed in the
 * slot since the block's H2D: the H2D is followed by the chunk digests of the slot's copy runs
 * on the prefetch stream (sh_block_digest), and the write-back compares them on the evict stream
 * and copies the changed runs (sh_saveback_submit_chunks). The host region ends up holding the slot's
 * bytes, as after the reference's full copy (engine.rs:232-262). 0: every byte is copied. */
int sh_turbo_set_writeback_chunks(sh_turbo* t, uint32_t chunk_bytes);
int sh_turbo_block_slot(sh_turbo* t, uint32_t block, int32_t* slot);     /* -1: none, engine.rs:375-378 */
int sh_turbo_block_location(sh_turbo* t, uint32_t block, int* location); /* engine.rs:384-393 */
int sh_turbo_counts(sh_turbo* t, uint32_t* blocks, uint32_t* slots, uint32_t* free_slots); /* engine.rs:380-382 */
/* Bytes moved so far in each direction (telemetry; no reference counterpart). */
int sh_turbo_bytes(sh_turbo* t, uint64_t* h2d, uint64_t* d2h);
/* Timing of later H2D copies (no reference counterpart): with timing on, each
 * block's latest H2D is bracketed by timing events; sh_turbo_block_times waits
 * for it and returns its start and end in ms after `ref_event` (a timing event
 * recorded earlier). */
int sh_turbo_set_timing(sh_turbo* t, int enable);
int sh_turbo_block_times(sh_turbo* t, uint32_t block, void* ref_event, float* out2);
/* Spans recorded since timing was last switched on (no reference counterpart),
 * on the HSA system clock of sh_saveback_clock_ns:
 *   SH_TURBO_SPAN_WRITEBACK  a block's write-back on the SDMA engine, from the
 *                            start of its first copy to the end of its last
 *                            (both 0 when a tool replaced the copies' signals);
 *   SH_TURBO_SPAN_HOST_WAIT  a host wait inside sh_turbo_step for the write-back
 *                            out of the slot or pinned region a prefetch reuses.
 * Waits for every recorded write-back first, copies up to `cap` spans to `out`
 * and sets *n to the number recorded. */
enum sh_turbo_span_kind { SH_TURBO_SPAN_WRITEBACK = 0, SH_TURBO_SPAN_HOST_WAIT = 1 };
typedef struct sh_turbo_span {
  uint32_t block, kind;
  uint64_t start_ns, end_ns;
  uint64_t bytes;  /* write-back bytes; 0 for a host wait */
} sh_turbo_span;
int sh_turbo_trace_spans(sh_turbo* t, sh_turbo_span* out, uint32_t cap, uint32_t* n);

/* ───────────────────────── VMM residency allocator ─────────────────────────
 * Slabs of reserved device address space whose regions get physical memory on
 * demand (hipMemCreate / hipMemMap / hipMemSetAccess) and lose it under a VRAM
 * ceiling: the HIP rewrite of the reference's SlabAllocator
 * (vmm_src/allocator.rs:75-713, eviction.rs:15-144, handle.rs:65-110,
 * prefetch.rs, Python surface vmm_src/python.rs:39-267). Thread-safe; a
 * Resident region is served with atomics only. Region offsets must be
 * multiples of the granularity and regions must fit their slab
 * (SH_ERR_INVALID otherwise). Each region reserves its own address range (a
 * slab groups its regions and bounds their offsets; regions of one slab are not
 * contiguous in address space): on gfx950, hipMemSetAccess refuses a mapping
 * inside a reservation that already holds a mapping of another size.
 * Errors (vmm_src/error.rs:30-53): Watermarked / NoEvictableRegions →
 * SH_ERR_WATERMARK (MemoryError); invalid slab / region → SH_ERR_INVALID
 * (ValueError); slab with live handles, released handle → SH_ERR_STATE
 * (RuntimeError); HIP failures → SH_ERR_HIP (RuntimeError). */
enum sh_vmm_region_state { SH_VMM_UNMAPPED = 0, SH_VMM_MAPPED_EMPTY = 1, SH_VMM_RESIDENT = 2 }; /* slab.rs:9-20 */
typedef struct sh_vmm sh_vmm;
typedef struct sh_vmm_handle sh_vmm_handle;
typedef struct sh_vmm_stats {  /* python.rs:97-106 */
  uint64_t total_slabs;
  uint64_t total_regions;
  uint64_t mapped_bytes;
  uint64_t vram_ceiling;
  uint64_t granularity;
  /* counters (no reference counterpart) */
  uint64_t maps;
  uint64_t evictions;
  uint64_t unmap_failures;
  uint64_t last_unmap_error;  /* hipError_t of the last failed unmap */
} sh_vmm_stats;
typedef struct sh_vmm_region_stats {  /* allocator.rs:51-58 */
  uint32_t state;
  uint32_t refcount;
  uint64_t offset;
  uint64_t size;
  uint64_t last_access;
  uint64_t watermark;  /* of the region's slab */
  uint32_t priority;   /* of the region's slab */
  uint32_t reserved;
} sh_vmm_region_stats;
/* ceiling_bytes 0: total VRAM - max(2 GB, 15 %) (allocator.rs:111-115). */
int sh_vmm_create(int device, uint64_t ceiling_bytes, sh_vmm** out);            /* allocator.rs:80-137 */
/* The allocator's memory is released once every handle is released too. */
int sh_vmm_destroy(sh_vmm* v);                                                  /* allocator.rs:648-713 */
int sh_vmm_info(sh_vmm* v, sh_vmm_stats* stats);                                /* allocator.rs:591-646 */
int sh_vmm_create_slab(sh_vmm* v, uint64_t size, uint32_t* slab);               /* allocator.rs:140-172 */
int sh_vmm_define_region(sh_vmm* v, uint32_t slab, uint64_t offset, uint64_t size, uint32_t* region); /* :175-198 */
int sh_vmm_ensure_resident(sh_vmm* v, uint32_t slab, uint32_t region, void* stream, sh_vmm_handle** out); /* :213-468 */
int sh_vmm_prefetch(sh_vmm* v, uint32_t slab, uint32_t region);                 /* allocator.rs:470-503 */
/* Times the fast path natively: out2[0] = ns per ensure_resident of a resident region (the
 * handles released after the timed loop), out2[1] = ns per ensure_resident + handle release
 * (which records an event on `stream`), each over `iters` calls. No reference counterpart:
 * it measures the operation the reference publishes as "ensure_resident (hot path) 250 ns
 * median" (README.md:165-170) without Python in the loop. */
int sh_vmm_time_fast_path(sh_vmm* v, uint32_t slab, uint32_t region, void* stream, uint32_t iters, double* out2);
int sh_vmm_set_priority(sh_vmm* v, uint32_t slab, uint32_t priority);          /* allocator.rs:505-533 */
int sh_vmm_set_ceiling(sh_vmm* v, uint64_t ceiling_bytes);                      /* allocator.rs:535-537 */
int sh_vmm_destroy_slab(sh_vmm* v, uint32_t slab);                              /* allocator.rs:539-585 */
int sh_vmm_region_info(sh_vmm* v, uint32_t slab, uint32_t region, sh_vmm_region_stats* stats);
int sh_vmm_handle_ptr(sh_vmm_handle* h, void** ptr);                            /* handle.rs:36-44 */
/* Mapping generation of the region when the handle was taken; it changes at
 * every (re)map, after which the region holds no data (no reference
 * counterpart: the reference's populate-once flag survives an eviction,
 * vmm_backend.py:205-208). */
int sh_vmm_handle_generation(sh_vmm_handle* h, uint64_t* generation);
/* Records an event on the handle's stream, then drops its reference
 * (handle.rs:65-110); SH_ERR_STATE when already released (python.rs:225-233). */
int sh_vmm_handle_release(sh_vmm_handle* h);
int sh_vmm_handle_destroy(sh_vmm_handle* h);  /* releases if needed, frees the handle */

/* DLPack (the open tensor-exchange ABI, DLManagedTensor layout) with the ROCm
 * device type, replacing vmm_src/dlpack.rs:4-76 (kDLCUDA). The exported tensor
 * holds its own reference to the region until its deleter runs
 * (python.rs:137-221). */
#define SH_DL_ROCM 10
typedef struct { int32_t device_type; int32_t device_id; } sh_dl_device;
typedef struct { uint8_t code; uint8_t bits; uint16_t lanes; } sh_dl_dtype;
typedef struct {
  void* data;
  sh_dl_device device;
  int32_t ndim;
  sh_dl_dtype dtype;
  int64_t* shape;
  int64_t* strides;
  uint64_t byte_offset;
} sh_dl_tensor;
typedef struct sh_dl_managed_tensor {
  sh_dl_tensor dl_tensor;
  void* manager_ctx;
  void (*deleter)(struct sh_dl_managed_tensor* self);
} sh_dl_managed_tensor;
int sh_vmm_handle_export(sh_vmm_handle* h, uint8_t code, uint8_t bits, int32_t ndim, const int64_t* shape,
                         sh_dl_managed_tensor** out);
/* Runs the deleter of an export that was never consumed. */
int sh_dl_free(sh_dl_managed_tensor* t);

/* Host copy of the kernels' row-index division (floor(n[i] / d) through the
 * 64-bit multiplicative inverse stored in sh_unpack_desc.div_magic), exported
 * so the index arithmetic can be checked on a CPU. No reference counterpart. */
int sh_index_div(uint32_t d, const uint32_t* n, uint32_t* q, size_t count);

#ifdef __cplusplus
}
#endif

#endif /* STAGEHAND_NATIVE_H */
