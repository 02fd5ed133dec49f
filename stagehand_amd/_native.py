"""ctypes binding of ``libstagehand_native.so`` (C ABI in ``include/stagehand_native.h``).

The library is loaded lazily on first use. A missing library is an error, not
a fallback: every product path that needs it raises :class:`NativeLibraryError`
telling how to build it.

Status codes map to the exception types the reference raises for the same
conditions (turbo_src/lib.rs:38-40 → RuntimeError, turbo_src/lib.rs:59-61 →
ValueError, src/stagehand/pool.py:133-139 → StagehandOOMError,
vmm_src/error.rs:30-53 → MemoryError for watermark refusals, and OSError for
weight-file reads, as the reference's open/mmap of a weight file raises).
"""
from __future__ import annotations

import atexit
import ctypes
import itertools
import logging
import threading
import weakref
from pathlib import Path

import numpy as np

from stagehand_amd.errors import StagehandOOMError

__all__ = [
    "NativeLibraryError",
    "track",
    "shutdown",
    "lib",
    "check",
    "LIB_PATH",
    "DESC_DTYPE",
    "PLAN_INFO_DTYPE",
    "SH_OK",
    "SH_ERR_NOT_READY",
    "KIND_I8_ROWSCALE_BF16",
    "KIND_I8_ROWSCALE_F32",
    "KIND_F32_BF16",
    "KIND_BF16_F32",
    "KIND_COPY_BYTES",
    "KIND_ZERO_BYTES",
]

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libstagehand_native.so"

SH_OK = 0
SH_ERR_INVALID = 1
SH_ERR_HIP = 2
SH_ERR_OOM = 3
SH_ERR_NOT_READY = 4
SH_ERR_STATE = 5
SH_ERR_TIMEOUT = 6
SH_ERR_WATERMARK = 7
SH_ERR_IO = 8

SH_FILE_DIRECT = 1
SH_FILE_ALIGN = 4096
SH_FILE_WILLNEED = 1
SH_FILE_DONTNEED = 2

KIND_I8_ROWSCALE_BF16 = 1
KIND_I8_ROWSCALE_F32 = 2
KIND_F32_BF16 = 3
KIND_BF16_F32 = 4
KIND_COPY_BYTES = 5
KIND_ZERO_BYTES = 6

# Mirror of `struct sh_unpack_desc` (64 bytes, little endian, natural alignment).
DESC_DTYPE = np.dtype(
    [
        ("src_off", "<u8"),
        ("dst_off", "<u8"),
        ("rows", "<u4"),
        ("cols", "<u4"),
        ("src_ld", "<u4"),
        ("kind", "<u4"),
        ("scale_off", "<u8"),
        ("div_magic", "<u8"),
        ("tile_begin", "<u4"),
        ("ntiles", "<u4"),
        ("lead", "<u4"),
        ("reserved", "<u4"),
    ]
)
assert DESC_DTYPE.itemsize == 64

# Mirror of `struct sh_plan_info`.
PLAN_INFO_DTYPE = np.dtype(
    [
        ("n_desc", "<u4"),
        ("n_tiles", "<u4"),
        ("kind_mask", "<u4"),
        ("tile_elems", "<u4"),
        ("src_extent", "<u8"),
        ("dst_extent", "<u8"),
        ("scale_extent", "<u8"),
        ("algo_bytes", "<u8"),
        ("elements", "<u8"),
    ]
)


class NativeLibraryError(RuntimeError):
    """The native library is missing or does not match this package."""


_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_i32 = ctypes.c_int
_u32 = ctypes.c_uint32

# name → argtypes; every function returns int status.
_SIGNATURES: dict[str, list] = {
    "sh_abi_version": [],
    "sh_unpack_noalloc": [_vp, _u32, _vp, _sz, _vp, _vp, _sz, _vp, _sz, _vp],
    "sh_shutdown": [_vp],
    "sh_device_count": [ctypes.POINTER(_i32)],
    "sh_set_device": [_i32],
    "sh_get_device": [ctypes.POINTER(_i32)],
    "sh_host_alloc": [_sz, ctypes.POINTER(_vp)],
    "sh_host_free": [_vp],
    "sh_stream_create": [ctypes.POINTER(_vp)],
    "sh_stream_destroy": [_vp],
    "sh_stream_sync": [_vp],
    "sh_stream_wait_event": [_vp, _vp],
    "sh_event_create": [_i32, ctypes.POINTER(_vp)],
    "sh_event_destroy": [_vp],
    "sh_event_record": [_vp, _vp],
    "sh_event_query": [_vp],
    "sh_event_sync": [_vp],
    "sh_event_elapsed_ms": [_vp, _vp, ctypes.POINTER(ctypes.c_float)],
    "sh_memcpy_h2d_async": [_vp, _vp, _sz, _vp],
    "sh_memcpy_d2h_async": [_vp, _vp, _sz, _vp],
    "sh_memcpy_d2d_async": [_vp, _vp, _sz, _vp],
    "sh_plan_create": [_vp, _u32, ctypes.POINTER(_vp)],
    "sh_plan_destroy": [_vp],
    "sh_plan_get_info": [_vp, _vp],
    "sh_plan_describe": [_vp, _u32, _vp],
    "sh_index_div": [_u32, _vp, _vp, _sz],
    "sh_unpack": [_vp, _vp, _sz, _vp, _vp, _sz, _vp, _sz, _vp],
    "sh_dequant_i8_rowscale_bf16": [_vp, _vp, _sz, _vp, _vp, _sz, _vp, _sz, _vp],
    "sh_unpack_cast_f32_bf16": [_vp, _vp, _sz, _vp, _sz, _vp],
    "sh_pool_create": [_u32, ctypes.c_uint64, _i32, ctypes.POINTER(_vp)],
    "sh_pool_destroy": [_vp],
    "sh_pool_slab_ptr": [_vp, _u32, ctypes.POINTER(_vp)],
    "sh_pool_acquire": [_vp, ctypes.c_int64, ctypes.POINTER(_u32), ctypes.POINTER(ctypes.c_double)],
    "sh_pool_release": [_vp, _u32],
    "sh_pool_release_after": [_vp, _u32, _vp],
    "sh_pool_get_stats": [_vp, _vp],
    "sh_host_copy_batch": [_vp, _sz, _i32],
    "sh_file_open": [ctypes.c_char_p, _i32, ctypes.POINTER(_vp)],
    "sh_file_close": [_vp],
    "sh_file_get_info": [_vp, _vp],
    "sh_file_advise": [_vp, ctypes.c_uint64, ctypes.c_uint64, _i32],
    "sh_file_read_batch": [_vp, _sz, _vp, _i32],
    "sh_loader_create": [_vp, _i32, ctypes.POINTER(_vp)],
    "sh_loader_destroy": [_vp],
    "sh_loader_streams": [_vp, ctypes.POINTER(_vp), ctypes.POINTER(_vp)],
    "sh_loader_submit": [_vp, _vp, _vp, ctypes.POINTER(ctypes.c_uint64)],
    "sh_loader_query": [_vp, ctypes.c_uint64],
    "sh_loader_stream_wait": [_vp, ctypes.c_uint64, _vp],
    "sh_loader_sync": [_vp, ctypes.c_uint64],
    "sh_loader_query_copy": [_vp, ctypes.c_uint64],
    "sh_loader_sync_copy": [_vp, ctypes.c_uint64],
    "sh_loader_release": [_vp, ctypes.c_uint64],
    "sh_loader_set_timing": [_vp, _i32],
    "sh_loader_ticket_times": [_vp, ctypes.c_uint64, _vp, _vp],
    "sh_saveback_create": [_i32, ctypes.POINTER(_vp)],
    "sh_saveback_destroy": [_vp],
    "sh_saveback_submit": [_vp, _vp, ctypes.c_uint64, _vp, ctypes.POINTER(ctypes.c_uint64)],
    "sh_saveback_submit_after": [_vp, _vp, ctypes.c_uint64, _vp, _u32, ctypes.POINTER(ctypes.c_uint64)],
    "sh_saveback_query": [_vp, ctypes.c_uint64],
    "sh_saveback_wait": [_vp, ctypes.c_uint64],
    "sh_saveback_release": [_vp, ctypes.c_uint64],
    "sh_saveback_set_timing": [_vp, _i32],
    "sh_saveback_clock_ns": [ctypes.POINTER(ctypes.c_uint64)],
    "sh_saveback_ticket_times": [_vp, ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64)],
    "sh_saveback_submit_chunks": [_vp, _vp, _u32, _u32, _vp, _vp, _vp, _vp, _u32, _vp, ctypes.POINTER(ctypes.c_uint64)],
    "sh_saveback_ticket_bytes": [_vp, ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64)],
    "sh_block_digest": [_vp, ctypes.c_uint64, _u32, _vp, _vp],
    "sh_block_changed": [_vp, ctypes.c_uint64, _u32, _vp, _vp, _vp],
    "sh_block_digest_host": [_vp, ctypes.c_uint64, _u32, _vp],
    "sh_turbo_create": [ctypes.POINTER(_vp)],
    "sh_turbo_destroy": [_vp],
    "sh_turbo_register_block": [_vp, _vp, _u32, ctypes.POINTER(_u32)],
    "sh_turbo_initialize": [_vp, _i32, _u32],
    "sh_turbo_set_save_back": [_vp, _i32],
    "sh_turbo_stage_block": [_vp, _u32, _vp, _u32],
    "sh_turbo_step": [_vp, _u32, _i32, _vp],
    "sh_turbo_evict_sync": [_vp, _u32, _vp],
    "sh_turbo_drain": [_vp],
    "sh_turbo_gpu_ptr": [_vp, _u32, _u32, ctypes.POINTER(ctypes.c_uint64)],
    "sh_turbo_cpu_ptr": [_vp, _u32, _u32, ctypes.POINTER(ctypes.c_uint64)],
    "sh_turbo_param_offset": [_vp, _u32, _u32, ctypes.POINTER(ctypes.c_uint64)],
    "sh_turbo_set_slot_gpu_ptrs": [_vp, _u32, _vp, _u32],
    "sh_turbo_set_slot_buffer": [_vp, _u32, _vp, ctypes.c_uint64],
    "sh_turbo_slot_bytes": [_vp, ctypes.POINTER(ctypes.c_uint64)],
    "sh_turbo_set_writeback": [_vp, _u32, _i32],
    "sh_turbo_block_slot": [_vp, _u32, ctypes.POINTER(ctypes.c_int32)],
    "sh_turbo_block_location": [_vp, _u32, ctypes.POINTER(_i32)],
    "sh_turbo_counts": [_vp, ctypes.POINTER(_u32), ctypes.POINTER(_u32), ctypes.POINTER(_u32)],
    "sh_turbo_bytes": [_vp, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)],
    "sh_turbo_set_timing": [_vp, _i32],
    "sh_vmm_create": [_i32, ctypes.c_uint64, ctypes.POINTER(_vp)],
    "sh_vmm_destroy": [_vp],
    "sh_vmm_time_fast_path": [_vp, _u32, _u32, _vp, _u32, _vp],
    "sh_vmm_info": [_vp, _vp],
    "sh_vmm_create_slab": [_vp, ctypes.c_uint64, ctypes.POINTER(_u32)],
    "sh_vmm_define_region": [_vp, _u32, ctypes.c_uint64, ctypes.c_uint64, ctypes.POINTER(_u32)],
    "sh_vmm_ensure_resident": [_vp, _u32, _u32, _vp, ctypes.POINTER(_vp)],
    "sh_vmm_prefetch": [_vp, _u32, _u32],
    "sh_vmm_set_priority": [_vp, _u32, _u32],
    "sh_vmm_set_ceiling": [_vp, ctypes.c_uint64],
    "sh_vmm_destroy_slab": [_vp, _u32],
    "sh_vmm_region_info": [_vp, _u32, _u32, _vp],
    "sh_vmm_handle_ptr": [_vp, ctypes.POINTER(_vp)],
    "sh_vmm_handle_generation": [_vp, ctypes.POINTER(ctypes.c_uint64)],
    "sh_vmm_handle_release": [_vp],
    "sh_vmm_handle_destroy": [_vp],
    "sh_vmm_handle_export": [_vp, ctypes.c_uint8, ctypes.c_uint8, ctypes.c_int32, _vp, ctypes.POINTER(_vp)],
    "sh_dl_free": [_vp],
    "sh_turbo_block_times": [_vp, _u32, _vp, _vp],
    "sh_turbo_trace_spans": [_vp, _vp, _u32, _vp],
    "sh_turbo_set_writeback_chunks": [_vp, _u32],
}

# Mirror of `struct sh_chunk_region`.
CHUNK_REGION_DTYPE = np.dtype([("host_dst", "<u8"), ("dev_src", "<u8"), ("bytes", "<u8"), ("first_chunk", "<u8")])

# Mirror of `struct sh_load_request`.
LOAD_REQUEST_DTYPE = np.dtype([
    ("pieces", "<u8"), ("n_pieces", "<u8"), ("src_bytes", "<u8"), ("plan", "<u8"), ("staging", "<u8"),
    ("staging_bytes", "<u8"), ("dst", "<u8"), ("dst_bytes", "<u8"), ("scale_off", "<i8"), ("zp_off", "<i8"),
    ("n_scale", "<u8"), ("copy_threads", "<i4"), ("reserved", "<i4"), ("image", "<u8"),
    ("ranges", "<u8"), ("n_ranges", "<u8"), ("dma", "<u8"), ("n_dma", "<u8"), ("wait_event", "<u8"),
    ("saveback", "<u8"), ("saveback_ticket", "<u8"), ("digest", "<u8"), ("digest_bytes", "<u8"),
    ("digest_chunk", "<u4"), ("reserved2", "<u4"),
])

# Mirrors of `struct sh_file_range` / `struct sh_file_info`.
FILE_RANGE_DTYPE = np.dtype([("file", "<u8"), ("file_off", "<u8"), ("bytes", "<u8"), ("dst", "<u8")])
FILE_INFO_DTYPE = np.dtype([("size", "<u8"), ("direct", "<u8"), ("bytes_direct", "<u8"), ("bytes_bounced", "<u8"),
                            ("bytes_buffered", "<u8"), ("bytes_cached", "<u8"), ("reads", "<u8")])

# Mirror of `struct sh_pool_stats`.
POOL_STATS_DTYPE = np.dtype([
    ("total", "<u8"), ("free", "<u8"), ("in_use", "<u8"), ("peak_in_use", "<u8"), ("wait_count", "<u8"),
    ("fenced", "<u8"), ("total_wait_ms", "<f8"), ("slab_bytes", "<u8"), ("pinned", "<u8"),
])

# Mirrors of `struct sh_vmm_stats` / `struct sh_vmm_region_stats`.
VMM_STATS_DTYPE = np.dtype([("total_slabs", "<u8"), ("total_regions", "<u8"), ("mapped_bytes", "<u8"),
                            ("vram_ceiling", "<u8"), ("granularity", "<u8"), ("maps", "<u8"), ("evictions", "<u8"),
                            ("unmap_failures", "<u8"), ("last_unmap_error", "<u8")])
VMM_REGION_DTYPE = np.dtype([("state", "<u4"), ("refcount", "<u4"), ("offset", "<u8"), ("size", "<u8"),
                             ("last_access", "<u8"), ("watermark", "<u8"), ("priority", "<u4"), ("reserved", "<u4")])

# Mirror of `struct sh_copy_item`.
COPY_ITEM_DTYPE = np.dtype([("dst", "<u8"), ("src", "<u8"), ("bytes", "<u8")])
TURBO_SPAN_DTYPE = np.dtype([("block", "<u4"), ("kind", "<u4"), ("start_ns", "<u8"), ("end_ns", "<u8"),
                             ("bytes", "<u8")])
TURBO_SPAN_WRITEBACK, TURBO_SPAN_HOST_WAIT = 0, 1

ABI_VERSION = 8

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def exported_symbols() -> list[str]:
    """Names of every C entry point this binding expects the library to export."""
    return sorted(_SIGNATURES) + ["sh_last_error"]


def lib() -> ctypes.CDLL:
    """Return the loaded native library, loading it on first use."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise NativeLibraryError(
                f"{LIB_PATH} is not built; run `python -m stagehand_amd.build_native` "
                "(or __graft_entry__.build()) first"
            )
        handle = ctypes.CDLL(str(LIB_PATH))
        handle.sh_last_error.restype = ctypes.c_char_p
        handle.sh_last_error.argtypes = []
        for name, argtypes in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = ctypes.c_int
            fn.argtypes = argtypes
        got = handle.sh_abi_version()
        if got != ABI_VERSION:
            raise NativeLibraryError(f"{LIB_PATH} has ABI version {got}, expected {ABI_VERSION}; rebuild it")
        _lib = handle
        return _lib


def last_error() -> str:
    msg = lib().sh_last_error()
    return msg.decode(errors="replace") if msg else ""


def check(status: int, what: str = "") -> int:
    """Raise the mapped Python exception for a failed native status."""
    if status == SH_OK or status == SH_ERR_NOT_READY:
        return status
    msg = last_error() or f"{what} failed with status {status}"
    if status == SH_ERR_INVALID:
        raise ValueError(msg)
    if status == SH_ERR_OOM:
        raise StagehandOOMError(msg)
    if status == SH_ERR_WATERMARK:
        raise MemoryError(msg)
    if status == SH_ERR_TIMEOUT:
        raise TimeoutError(msg)
    if status == SH_ERR_IO:
        raise OSError(msg)
    raise RuntimeError(msg)


def call(name: str, *args) -> int:
    """Call native entry point *name* and raise on failure."""
    return check(getattr(lib(), name)(*args), name)


# ── process teardown ─────────────────────────────────────────────────────────
#
# Native objects own threads (loader workers and advisors, save-back workers, the VMM
# prefetch worker, the shared host copy threads), HIP streams, events and pinned memory.
# Objects still open when the interpreter exits are closed by ``shutdown`` (registered
# with atexit on first use), while the HIP runtime is still whole: users before what they
# use — runtimes, then engines, then what engines hold — and sh_shutdown last.

CLOSE_RUNTIME, CLOSE_ENGINE_USER, CLOSE_ENGINE, CLOSE_LEAF, CLOSE_POOL = range(5)

log = logging.getLogger(__name__)


class _LiveCounts(ctypes.Structure):
    _fields_ = [(name, ctypes.c_uint64) for name in
                ("pools", "loaders", "savebacks", "turbos", "vmms", "files", "copy_threads",
                 "kernel_devices")]


_tracked: list[tuple[int, int, weakref.ref, str]] = []
_tracked_lock = threading.Lock()
_tracked_seq = itertools.count()
_atexit_registered = False


def track(obj: object, order: int, method: str = "close") -> None:
    """Closes ``obj`` with ``obj.<method>()`` at interpreter exit if it is still alive then.
    Objects close in ``order`` (CLOSE_RUNTIME first), the newest first within one order."""
    global _atexit_registered
    with _tracked_lock:
        if len(_tracked) >= 1024:
            _tracked[:] = [t for t in _tracked if t[2]() is not None]
        _tracked.append((order, next(_tracked_seq), weakref.ref(obj), method))
        if not _atexit_registered:
            atexit.register(shutdown)
            _atexit_registered = True


def shutdown() -> dict[str, int]:
    """Closes every tracked native object that is still alive, then ends the library's
    process-wide state (``sh_shutdown``: the shared copy threads are joined and the kernels'
    code is unloaded). Returns the native objects still alive afterwards, by kind (all zero
    when everything closed)."""
    with _tracked_lock:
        items = sorted(_tracked, key=lambda t: (t[0], -t[1]))
        _tracked.clear()
    for _order, _seq, ref, method in items:
        obj = ref()
        if obj is None:
            continue
        try:
            getattr(obj, method)()
        except Exception as exc:  # noqa: BLE001 — keep closing the rest
            log.warning("stagehand shutdown: %s.%s() failed: %s", type(obj).__name__, method, exc)
    if _lib is None:
        return {}
    counts = _LiveCounts()
    check(_lib.sh_shutdown(ctypes.byref(counts)), "sh_shutdown")
    out = {name: int(getattr(counts, name)) for name, _ in _LiveCounts._fields_}
    left = {k: v for k, v in out.items() if v}
    if left:
        log.warning("stagehand shutdown: native objects still alive: %s", left)
    return out
