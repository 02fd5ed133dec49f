"""Async H2D/D2H transfers and native block loads.

``AsyncTransferEngine`` keeps the contract of src/stagehand/transfer.py:69-314
— ``submit_h2d`` / ``submit_d2h`` / ``poll`` / ``wait`` / ``inflight_count`` /
``reap`` / ``drain`` with ``max_inflight`` backpressure and a
``TransferHandle`` carrying the same fields — but its copies are
``hipMemcpyAsync`` calls on a native copy stream fenced by native events
(include/stagehand_native.h), and it adds the device path the scheduler uses
for whole blocks:

* ``submit_block_load`` hands a block's source pieces to the native loader
  (a worker thread: gather into a pinned slab, H2D on the copy stream; the
  unpack kernel then runs on the stream that first waits for the load, or on
  the loader's unpack stream when the host waits first), returning immediately;
* ``wait_device`` makes the caller's current stream wait for a transfer on the
  device, without blocking the host (the reference's ``wait`` blocks the host
  in ``event.synchronize()``, src/stagehand/transfer.py:203; ``wait`` here keeps
  that behaviour for callers that need it).

Without a GPU, copies are synchronous ``copy_`` calls and handles complete at
submission, as in the reference (src/stagehand/transfer.py:136-138).
"""
from __future__ import annotations

import ctypes
import logging
import os
import threading
import time
from collections import Counter
from contextlib import contextmanager
from dataclasses import dataclass, field
from typing import TYPE_CHECKING, Any

import numpy as np
import torch

from stagehand_amd import _native
from stagehand_amd._native import COPY_ITEM_DTYPE, FILE_RANGE_DTYPE, LOAD_REQUEST_DTYPE
from stagehand_amd.errors import TransferError

if TYPE_CHECKING:
    from stagehand_amd.pool import PinnedPool, PinnedSlab
    from stagehand_amd.unpack import UnpackPlan

__all__ = ["TransferHandle", "AsyncTransferEngine", "NativeEvent", "BlockSource", "SaveBackEngine", "SaveBackTicket"]

log = logging.getLogger(__name__)
_STALL_LOGS_ENABLED = str(os.getenv("SERENITY_STAGEHAND_STALL_LOGS", "0")).strip().lower() in {"1", "true", "yes", "on"}


class NativeEvent:
    """A native HIP event with the ``query``/``synchronize`` face of ``torch.cuda.Event``."""

    def __init__(self, timing: bool = False) -> None:
        h = ctypes.c_void_p()
        _native.call("sh_event_create", int(timing), ctypes.byref(h))
        self.handle = h

    def elapsed_ms(self, later: "NativeEvent") -> float:
        ms = ctypes.c_float()
        _native.call("sh_event_elapsed_ms", self.handle, later.handle, ctypes.byref(ms))
        return ms.value

    def record(self, stream_handle: int) -> None:
        _native.call("sh_event_record", self.handle, stream_handle)

    def query(self) -> bool:
        return _native.call("sh_event_query", self.handle) == _native.SH_OK

    def synchronize(self) -> None:
        _native.call("sh_event_sync", self.handle)

    def wait_on(self, stream_handle: int) -> None:
        """Makes ``stream_handle`` wait for this event on the device."""
        _native.call("sh_stream_wait_event", stream_handle, self.handle)

    def __del__(self) -> None:
        try:
            if self.handle is not None:
                _native.lib().sh_event_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


class SaveBackEngine:
    """Device→host save-back copies on an SDMA engine (native ``sh_saveback``).

    The reference copies an evicted block's parameters back with a synchronous
    ``param.data.to("cpu")`` (src/stagehand/scheduler.py:1216-1226, 1348-1366).
    ``hipMemcpyAsync`` would run these pinned device→host copies as kernels on
    the compute units, which slows the compute kernels running beside them; the
    SDMA engines copy without them. Each submission is ordered after the work
    queued on a stream (a worker thread waits for an event recorded there) and
    completes as a :class:`SaveBackTicket`; tickets complete in order.
    """

    def __init__(self, device: int) -> None:
        h = ctypes.c_void_p()
        _native.call("sh_saveback_create", int(device), ctypes.byref(h))
        self._h: ctypes.c_void_p | None = h
        self._timing = False
        _native.track(self, _native.CLOSE_LEAF)

    @property
    def handle(self) -> ctypes.c_void_p:
        if self._h is None:
            raise RuntimeError("the save-back engine has been shut down")
        return self._h

    @property
    def closed(self) -> bool:
        return self._h is None

    def submit(self, items: np.ndarray, stream_handle: int) -> "SaveBackTicket":
        """Copies ``items`` (COPY_ITEM_DTYPE rows: pinned host dst, device src, bytes) after the
        work queued so far on ``stream_handle``."""
        ticket = ctypes.c_uint64()
        _native.call("sh_saveback_submit", self.handle, items.ctypes.data if len(items) else None, len(items),
                     stream_handle, ctypes.byref(ticket))
        return SaveBackTicket(self, ticket.value)

    def submit_after(self, items: np.ndarray, events: "list[NativeEvent]") -> "SaveBackTicket":
        """Copies ``items`` once each of ``events`` has completed (the caller keeps them alive and
        unrecorded until the ticket completes)."""
        ticket = ctypes.c_uint64()
        handles = (ctypes.c_void_p * max(1, len(events)))(*[ev.handle.value for ev in events])
        _native.call("sh_saveback_submit_after", self.handle, items.ctypes.data if len(items) else None, len(items),
                     handles, len(events), ctypes.byref(ticket))
        return SaveBackTicket(self, ticket.value)

    def submit_chunks(self, regions: "list[tuple[int, int, int]]", chunk: int, digests: int, changed: int,
                      digest_stream: int, events: "list[NativeEvent] | None", stream_handle: int) -> "SaveBackTicket":
        """Copies the chunks of each region (pinned host dst, device src, bytes) whose digest differs
        from ``digests`` (device pointer, the regions' chunks one after another; 0 copies every
        chunk), after ``events`` (or after the work queued so far on ``stream_handle``): the worker
        compares them on ``digest_stream`` into ``changed`` (pinned, one byte per chunk). Every
        buffer stays in use until the ticket completes."""
        table = np.zeros(len(regions), dtype=_native.CHUNK_REGION_DTYPE)
        first = 0
        for i, (dst, src, nbytes) in enumerate(regions):
            table[i] = (dst, src, nbytes, first)
            first += -(-nbytes // chunk)
        ticket = ctypes.c_uint64()
        evs = events or []
        handles = (ctypes.c_void_p * max(1, len(evs)))(*[ev.handle.value for ev in evs])
        _native.call("sh_saveback_submit_chunks", self.handle, table.ctypes.data if len(table) else None, len(table),
                     chunk, digests or None, changed or None, digest_stream, handles if evs else None, len(evs),
                     stream_handle, ctypes.byref(ticket))
        return SaveBackTicket(self, ticket.value, counts_bytes=True)

    def set_timing(self, enable: bool) -> None:
        _native.call("sh_saveback_set_timing", self.handle, int(enable))
        self._timing = bool(enable)

    @staticmethod
    def clock_ns() -> int:
        ns = ctypes.c_uint64()
        _native.call("sh_saveback_clock_ns", ctypes.byref(ns))
        return ns.value

    def close(self) -> None:
        if self._h is not None:
            h, self._h = self._h, None
            _native.call("sh_saveback_destroy", h)

    def __del__(self) -> None:  # pragma: no cover - interpreter shutdown order
        try:
            self.close()
        except Exception:
            pass


class SaveBackTicket:
    """Completion of one :class:`SaveBackEngine` submission, with the ``query`` /
    ``synchronize`` face of :class:`NativeEvent`. It has no device-side form:
    ``wait_on`` waits on the host, and a load that reads what it wrote passes it as
    ``submit_block_load(wait_event=...)``, which the loader's worker waits for."""

    def __init__(self, engine: SaveBackEngine, ticket: int, counts_bytes: bool = False) -> None:
        self.engine = engine
        self.ticket = ticket
        # a chunk save-back: its copies (and so its bytes) are known once it completes
        self.counts_bytes = counts_bytes

    def query(self) -> bool:
        if self.engine.closed:  # closing the engine waited for every copy
            return True
        return _native.call("sh_saveback_query", self.engine.handle, self.ticket) == _native.SH_OK

    def synchronize(self) -> None:
        if not self.engine.closed:
            _native.call("sh_saveback_wait", self.engine.handle, self.ticket)

    def wait_on(self, stream_handle: int) -> None:
        """Waits on the host (the copy engine's completion has no device-side wait)."""
        self.synchronize()

    def copied_bytes(self) -> int:
        """Waits for the ticket; the bytes its copies moved."""
        out = ctypes.c_uint64()
        _native.call("sh_saveback_ticket_bytes", self.engine.handle, self.ticket, ctypes.byref(out))
        return out.value

    def times_ns(self) -> tuple[int, int]:
        out = (ctypes.c_uint64 * 2)()
        _native.call("sh_saveback_ticket_times", self.engine.handle, self.ticket, out)
        return out[0], out[1]

    def __del__(self) -> None:
        try:
            if not self.engine.closed:
                _native.lib().sh_saveback_release(self.engine.handle, ctypes.c_uint64(self.ticket))
        except Exception:
            pass


@dataclass
class TransferHandle:
    """Returned by every submit (fields of src/stagehand/transfer.py:32-42)."""

    handle_id: int
    block_id: str
    direction: str  # "h2d", "d2h" or "load"
    event: Any  # NativeEvent | None
    submitted_at: float
    size_bytes: int
    completed: bool = False
    ticket: int | None = None
    keepalive: list = field(default_factory=list, repr=False)
    device_waited: bool = False
    host_clock: bool = False  # submitted_at is on time.perf_counter (set while a trace runs)
    copy_landed: bool = False  # a block load's copies have landed (its unpack / digests may not have run)


@dataclass
class BlockSource:
    """What one block load sends: slab pieces (offset, host tensor or
    :class:`~stagehand_amd.fileio.FileRange`), the bytes to send, and optionally
    an unpack plan with the offsets of its scales."""

    pieces: list[tuple[int, Any]]
    src_bytes: int
    plan: "UnpackPlan | None" = None
    scale_off: int = -1
    zp_off: int = -1
    n_scale: int = 0
    # pinned-image caching: a layout signature, and the pieces whose bytes may
    # change between loads (module parameters); None key = not cacheable
    key: bytes | None = None
    mutable: frozenset = frozenset()


def _current_stream_handle() -> int:
    return torch.cuda.current_stream().cuda_stream


class AsyncTransferEngine:
    """Copies between pinned slabs and device tensors on a dedicated stream."""

    def __init__(
        self,
        pool: PinnedPool,
        max_inflight: int = 2,
        copy_stream: torch.cuda.Stream | None = None,
        copy_threads: int | None = None,
        pin_sources: bool = False,
        save_back: str = "sdma",
    ) -> None:
        self._pool = pool
        # pin_sources: keep one pinned host image per cacheable block source and
        # DMA straight from it (no staging copy after the first load)
        self._pin_sources = pin_sources
        self._images: dict[str, tuple[bytes, int, int]] = {}  # block → (key, pinned ptr, bytes)
        self.pinned_image_bytes = 0
        self._max_inflight = max_inflight
        self._has_cuda = torch.cuda.is_available()
        self._lock = threading.Lock()
        self._cond = threading.Condition(self._lock)
        self._inflight: list[TransferHandle] = []
        self._next_handle_id = 0
        self._loader = None
        self._loader_stream = None
        self._owned_stream = None
        self._copy_stream = None
        self._copy_threads = copy_threads or min(16, os.cpu_count() or 1)
        # bytes actually sent host→device / device→host (a SquareQ block sends its
        # int8 source, not its bf16 size; telemetry keeps the reference's block sizes)
        self.bytes_h2d = 0
        self.bytes_d2h = 0
        # bytes handed to chunk save-backs (d2h_changed), before leaving out the unchanged chunks
        self.bytes_d2h_requested = 0
        self.loads = 0
        # save-back copies in flight: (completion event, device/host tensors they read or
        # write, device bytes their caller gave up with them)
        self._pending_d2h: list[tuple[Any, list, int]] = []
        self._releasing_bytes = 0
        # where save-back copies run: "sdma" (SaveBackEngine) or "stream" (the copy stream)
        if save_back not in ("sdma", "stream"):
            raise ValueError(f"save_back must be 'sdma' or 'stream', got {save_back!r}")
        self._save_back = save_back
        self._saveback: SaveBackEngine | None = None
        self._trace_t0_ns = 0
        self._trace_t0_host = 0.0
        self._trace_waits: list[tuple[str, float, float]] = []
        # host time spent waiting, by kind (ms): see host_wait
        self.host_wait_ms: Counter = Counter()
        # optional device timeline (start_trace / stop_trace)
        self._trace_ref: NativeEvent | None = None
        self._trace_loads: list[tuple[str, int, float, float, float]] = []
        self._trace_compute: list[tuple[str, NativeEvent, NativeEvent]] = []
        _native.track(self, _native.CLOSE_ENGINE, "shutdown")
        if self._has_cuda:
            _native.call("sh_set_device", torch.cuda.current_device())
            if copy_stream is not None:
                self._copy_stream = copy_stream
            else:
                h = ctypes.c_void_p()
                _native.call("sh_stream_create", ctypes.byref(h))
                self._owned_stream = h
                self._copy_stream = torch.cuda.ExternalStream(h.value)

    # ── properties ───────────────────────────────────────────────────

    @property
    def copy_stream(self):
        return self._copy_stream

    @property
    def pool(self) -> PinnedPool:
        return self._pool

    def _loader_handle(self) -> ctypes.c_void_p:
        if self._loader is None:
            if self._pool.handle is None:
                raise RuntimeError("the pinned pool has been shut down")
            h = ctypes.c_void_p()
            _native.call("sh_loader_create", self._pool.handle, self._copy_threads, ctypes.byref(h))
            self._loader = h
        return self._loader

    def loader_streams(self) -> tuple[int, int]:
        cs, us = ctypes.c_void_p(), ctypes.c_void_p()
        _native.call("sh_loader_streams", self._loader_handle(), ctypes.byref(cs), ctypes.byref(us))
        return cs.value, us.value

    def _loader_unpack_stream(self) -> int:
        """The loader's unpack stream (hipStream_t value): where save-back chunk comparisons run
        (a load's own digests run where its post-copy work is queued: the waiting stream, or this
        one when the host waits)."""
        return self.loader_streams()[1]

    def _loader_copy_stream(self) -> torch.cuda.ExternalStream:
        if self._loader_stream is None:
            self._loader_stream = torch.cuda.ExternalStream(self.loader_streams()[0])
        return self._loader_stream

    def alloc_device(self, numel: int, dtype: torch.dtype) -> torch.Tensor:
        """A destination buffer for block loads, allocated on the loader's copy stream.

        torch's caching allocator hands a buffer freed on a stream back only to
        allocations on the same stream, after the work queued there; buffers from
        this pool are written by the loader's copy stream, so a load into one needs
        no wait on the compute stream's queue. Compute use must be registered with
        ``record_stream``, which keeps the memory from being handed out again until
        that compute has run: callers call ``record_stream`` on the buffer for every
        stream that uses it (the scheduler does so in ``before_block``)."""
        with torch.cuda.stream(self._loader_copy_stream()):
            return torch.empty(numel, dtype=dtype, device="cuda")

    # ── reference-compatible copies ──────────────────────────────────

    def submit_h2d(self, block_id: str, host_slab: PinnedSlab, gpu_dest: torch.Tensor) -> TransferHandle:
        size = gpu_dest.numel() * gpu_dest.element_size()
        self._wait_for_slot()
        handle = self._make_handle(block_id, "h2d", size)
        if self._has_cuda:
            if size > host_slab.size_bytes:
                raise TransferError(f"H2D of {size} bytes from a {host_slab.size_bytes}-byte slab")
            cs = self._copy_stream.cuda_stream
            self._fence_copy_stream(cs)
            self._check_copy(_native.lib().sh_memcpy_h2d_async(gpu_dest.data_ptr(), host_slab.buffer.data_ptr(), size, cs),
                             block_id, "h2d")
            handle.event = NativeEvent()
            handle.event.record(cs)
            handle.keepalive = [gpu_dest]
            self.bytes_h2d += size
        else:
            gpu_dest.view(-1).view(torch.uint8).copy_(host_slab.buffer[:size])
            handle.completed = True
        with self._lock:
            self._inflight.append(handle)
        return handle

    def submit_d2h(self, block_id: str, gpu_src: torch.Tensor, host_slab: PinnedSlab) -> TransferHandle:
        size = gpu_src.numel() * gpu_src.element_size()
        self._wait_for_slot()
        handle = self._make_handle(block_id, "d2h", size)
        if self._has_cuda:
            if size > host_slab.size_bytes:
                raise TransferError(f"D2H of {size} bytes into a {host_slab.size_bytes}-byte slab")
            cs = self._copy_stream.cuda_stream
            self._fence_copy_stream(cs)
            self._check_copy(_native.lib().sh_memcpy_d2h_async(host_slab.buffer.data_ptr(), gpu_src.data_ptr(), size, cs),
                             block_id, "d2h")
            handle.event = NativeEvent()
            handle.event.record(cs)
            handle.keepalive = [gpu_src]
            self.bytes_d2h += size
        else:
            host_slab.buffer[:size].copy_(gpu_src.reshape(-1).view(torch.uint8))
            handle.completed = True
        with self._lock:
            self._inflight.append(handle)
        return handle

    # ── native block loads ───────────────────────────────────────────

    def submit_block_load(self, block_id: str, source: BlockSource, gpu_dest: torch.Tensor,
                          dest_on_loader_stream: bool = False, wait_event: "NativeEvent | SaveBackTicket | None" = None,
                          pinned_pieces: bool = False,
                          digest: "tuple[torch.Tensor, int, int] | None" = None) -> TransferHandle:
        """Stage ``source`` into a pinned slab and land it in ``gpu_dest`` (device path).

        The copy waits for the work queued on the current stream (``gpu_dest`` may reuse
        memory that queued kernels still read) unless ``gpu_dest`` came from
        ``alloc_device`` (``dest_on_loader_stream``). With ``pinned_pieces`` (or a ``wait_event``),
        pieces that are pinned host tensors are copied straight to the device, with no slab and no
        host copy, so they are read until the load completes and must not change before then (the
        handle keeps them alive; asking each piece whether it is pinned costs a runtime query, so
        callers whose pieces are never pinned leave it off);
        ``wait_event`` (such as the save-back copy that wrote them) orders every copy after it: on
        the device for a :class:`NativeEvent`, on the loader's worker thread for a
        :class:`SaveBackTicket`. ``digest`` = (device tensor of 2 uint64 per chunk, bytes, chunk
        bytes): the chunk digests of ``gpu_dest``'s first bytes are written there once the load
        has landed, before it counts as done (for :meth:`d2h_changed`)."""
        if not self._has_cuda:
            raise RuntimeError("submit_block_load needs a GPU")
        dst_bytes = gpu_dest.numel() * gpu_dest.element_size()
        self._wait_for_slot()
        handle = self._make_handle(block_id, "load", source.src_bytes)
        image = 0
        pieces = source.pieces
        if self._pin_sources and source.key is not None and source.src_bytes > 0:
            image, fresh = self._image_for(block_id, source)
            if not fresh:
                pieces = [p for i, p in enumerate(source.pieces) if i in source.mutable]
        tensors = [(off, t) for off, t in pieces if isinstance(t, torch.Tensor)]
        files = [(off, t) for off, t in pieces if not isinstance(t, torch.Tensor)]
        for i, (_off, t) in enumerate(tensors):
            if t.device.type != "cpu" or not t.is_contiguous():
                raise ValueError(f"block {block_id}: piece {i} must be a contiguous host tensor")
        check = pinned_pieces or wait_event is not None
        pinned = [check and t.is_pinned() for _off, t in tensors]
        items = np.zeros(len(tensors) - sum(pinned), dtype=COPY_ITEM_DTYPE)
        dma = np.zeros(sum(pinned), dtype=COPY_ITEM_DTYPE)
        keep: list = [gpu_dest]
        ni = nd = 0
        for (off, t), pin in zip(tensors, pinned):
            row = (off, t.data_ptr(), t.numel() * t.element_size())
            if pin:
                dma[nd] = row
                nd += 1
            else:
                items[ni] = row
                ni += 1
            keep.append(t)
        if len(dma) > 1:
            # pieces contiguous both in the source slab and in host memory become one copy
            dma = np.sort(dma, order="dst")
            merged = [dma[0].copy()]
            for row in dma[1:]:
                last = merged[-1]
                if last["dst"] + last["bytes"] == row["dst"] and last["src"] + last["bytes"] == row["src"]:
                    last["bytes"] += row["bytes"]
                else:
                    merged.append(row.copy())
            dma = np.array(merged, dtype=COPY_ITEM_DTYPE)
        keep += [items, dma]
        if wait_event is not None:
            keep.append(wait_event)
        ranges = np.zeros(len(files), dtype=FILE_RANGE_DTYPE)
        for i, (off, fr) in enumerate(files):
            ranges[i] = (fr.file.handle, fr.offset, fr.nbytes, off)
            keep.append(fr.file)
        keep.append(ranges)
        req = np.zeros(1, dtype=LOAD_REQUEST_DTYPE)
        req[0]["pieces"] = items.ctypes.data
        req[0]["n_pieces"] = len(items)
        req[0]["src_bytes"] = source.src_bytes
        req[0]["dst"] = gpu_dest.data_ptr()
        req[0]["dst_bytes"] = dst_bytes
        req[0]["scale_off"] = source.scale_off
        req[0]["zp_off"] = source.zp_off
        req[0]["n_scale"] = source.n_scale
        req[0]["copy_threads"] = self._copy_threads
        req[0]["image"] = image
        req[0]["ranges"] = ranges.ctypes.data if len(ranges) else 0
        req[0]["n_ranges"] = len(ranges)
        req[0]["dma"] = dma.ctypes.data if len(dma) else 0
        req[0]["n_dma"] = len(dma)
        if isinstance(wait_event, SaveBackTicket):
            req[0]["saveback"] = wait_event.engine.handle.value
            req[0]["saveback_ticket"] = wait_event.ticket
        elif wait_event is not None:
            req[0]["wait_event"] = wait_event.handle.value
        if digest is not None:
            dig, nbytes, chunk = digest
            if nbytes > dst_bytes or dig.numel() * dig.element_size() < 16 * (-(-nbytes // chunk)):
                raise ValueError(f"block {block_id}: digest buffer too small for {nbytes} bytes in chunks of {chunk}")
            req[0]["digest"] = dig.data_ptr()
            req[0]["digest_bytes"] = nbytes
            req[0]["digest_chunk"] = chunk
            keep.append(dig)
        if source.plan is not None:
            if dest_on_loader_stream:
                with torch.cuda.stream(self._loader_copy_stream()):
                    staging = torch.empty(max(source.src_bytes, 1), dtype=torch.uint8, device=gpu_dest.device)
            else:
                staging = torch.empty(max(source.src_bytes, 1), dtype=torch.uint8, device=gpu_dest.device)
            keep.append(staging)
            keep.append(source.plan)
            req[0]["plan"] = source.plan.handle.value
            req[0]["staging"] = staging.data_ptr()
            req[0]["staging_bytes"] = staging.numel()
        ticket = ctypes.c_uint64()
        wait_stream = self.loader_streams()[0] if dest_on_loader_stream else _current_stream_handle()
        st = _native.lib().sh_loader_submit(self._loader_handle(), req.ctypes.data, wait_stream, ctypes.byref(ticket))
        if st != _native.SH_OK:
            self._raise_transfer(st, block_id, "load")
        handle.ticket = ticket.value
        handle.keepalive = keep
        if self._trace_ref is not None:
            handle.submitted_at, handle.host_clock = time.perf_counter(), True
        self.bytes_h2d += source.src_bytes
        self.loads += 1
        with self._lock:
            self._inflight.append(handle)
        return handle

    def _image_for(self, block_id: str, source: BlockSource) -> tuple[int, bool]:
        """Pinned image for ``block_id``; fresh=True when it must be filled with every piece."""
        hit = self._images.get(block_id)
        if hit is not None and hit[0] == source.key and hit[2] >= source.src_bytes:
            return hit[1], False
        if hit is not None:
            # the loader fences re-use of an image, not its release: drain before freeing
            self.drain()
            _native.call("sh_host_free", hit[1])
            self.pinned_image_bytes -= hit[2]
            del self._images[block_id]
        ptr = ctypes.c_void_p()
        _native.call("sh_host_alloc", source.src_bytes, ctypes.byref(ptr))
        self._images[block_id] = (source.key, ptr.value, source.src_bytes)
        self.pinned_image_bytes += source.src_bytes
        return ptr.value, True

    def free_images(self) -> None:
        if not self._images:
            return
        self.drain()
        if self._loader is not None:
            # every copy out of the images has completed once the loader's streams drain
            cs, us = self.loader_streams()
            _native.call("sh_stream_sync", cs)
            _native.call("sh_stream_sync", us)
        for _key, ptr, nbytes in self._images.values():
            _native.call("sh_host_free", ptr)
            self.pinned_image_bytes -= nbytes
        self._images.clear()

    # ── device timeline ──────────────────────────────────────────────

    def start_trace(self) -> None:
        """Time every later block load (copy start / copy end / done) and the compute
        spans the scheduler marks, relative to an event recorded now."""
        if not self._has_cuda:
            return
        _native.call("sh_loader_set_timing", self._loader_handle(), 1)
        sb = self._saveback_engine()
        if sb is not None:
            sb.set_timing(True)
        self._trace_ref = NativeEvent(timing=True)
        self._trace_ref.record(_current_stream_handle())
        # host times are aligned with the device timeline when the reference event completes
        self._trace_ref.synchronize()
        self._trace_t0_host = time.perf_counter()
        if sb is not None:
            # copy-engine times are read on the HSA system clock: take its value then too
            self._trace_t0_ns = sb.clock_ns()
        self._trace_loads = []
        self._trace_compute = []
        self._trace_d2h = []
        self._trace_waits = []

    @property
    def tracing(self) -> bool:
        return self._trace_ref is not None

    @contextmanager
    def host_wait(self, kind: str):
        """Accounts the host time spent in the block under ``kind`` (``host_wait_ms``); while a trace
        runs, also records the interval on the trace's timeline (ms after ``start_trace``)."""
        t0 = time.perf_counter()
        try:
            yield
        finally:
            t1 = time.perf_counter()
            self.host_wait_ms[kind] += (t1 - t0) * 1e3
            if self._trace_ref is not None:
                self._trace_waits.append((kind, (t0 - self._trace_t0_host) * 1e3, (t1 - self._trace_t0_host) * 1e3))

    def mark_compute(self, block_id: str, start: bool) -> None:
        if self._trace_ref is None:
            return
        ev = NativeEvent(timing=True)
        ev.record(_current_stream_handle())
        if start:
            self._trace_compute.append((block_id, ev, ev))
        else:
            for i in range(len(self._trace_compute) - 1, -1, -1):
                bid, s_ev, e_ev = self._trace_compute[i]
                if bid == block_id and e_ev is s_ev:
                    self._trace_compute[i] = (bid, s_ev, ev)
                    break

    def stop_trace(self) -> dict:
        """Drains and returns {"loads": [(block, bytes, start, copied, done) ms], "compute": [(block, start,
        end) ms], "d2h": [(bytes, start, end ms, "block" | "params"[, fence passed, host submit ms])]
        (save-back copies; SDMA ones also carry when the device passed the copy's fence, or None,
        and when the host submitted it)}."""
        if self._trace_ref is None:
            return {"loads": [], "compute": [], "d2h": []}
        self.drain()
        torch.cuda.synchronize()
        ref = self._trace_ref
        compute = [(bid, ref.elapsed_ms(s_ev), ref.elapsed_ms(e_ev)) for bid, s_ev, e_ev in self._trace_compute]
        d2h, untimed = [], 0
        for n, s_ev, e_ev, kind, *when in self._trace_d2h:
            if isinstance(s_ev, SaveBackTicket):  # copy-engine times, aligned at start_trace
                if n is None:  # a chunk save-back: the bytes of its changed chunks
                    n = s_ev.copied_bytes()
                    if n == 0:
                        continue
                try:
                    t0, t1 = s_ev.times_ns()
                except RuntimeError:  # a tool (a profiler's copy tracing) took the copies' signals
                    untimed += 1
                    continue
                # then: when the device passed the copy's fence (None when one of its events was
                # recorded before the trace, untimed), when the host submitted it
                fence_evs, submitted = when
                try:
                    fence_ms = max(ref.elapsed_ms(ev) for ev in fence_evs)
                except (RuntimeError, ValueError):
                    fence_ms = None
                d2h.append((n, (t0 - self._trace_t0_ns) / 1e6, (t1 - self._trace_t0_ns) / 1e6, kind,
                            fence_ms, (submitted - self._trace_t0_host) * 1e3))
            else:
                d2h.append((n, ref.elapsed_ms(s_ev), ref.elapsed_ms(e_ev), kind))
        out = {"loads": list(self._trace_loads), "compute": compute, "d2h": d2h, "d2h_untimed": untimed,
               "host_waits": list(self._trace_waits)}
        _native.call("sh_loader_set_timing", self._loader_handle(), 0)
        if self._saveback is not None:
            self._saveback.set_timing(False)
        self._trace_ref = None
        self._trace_loads, self._trace_compute, self._trace_d2h, self._trace_waits = [], [], [], []
        return out

    def _record_ticket_times(self, handle: TransferHandle) -> None:
        if self._trace_ref is None or handle.ticket is None:
            return
        out = (ctypes.c_float * 3)()
        st = _native.lib().sh_loader_ticket_times(self._loader, handle.ticket, self._trace_ref.handle, out)
        if st == _native.SH_OK:
            submit = (handle.submitted_at - self._trace_t0_host) * 1e3 if handle.host_clock else None
            self._trace_loads.append((handle.block_id, handle.size_bytes, out[0], out[1], out[2], submit))

    # ── asynchronous parameter save-back ─────────────────────────────

    def record_event(self) -> "NativeEvent | None":
        """An event recorded now on the current stream (None without a GPU): a save-back fence.
        Timed while a trace runs, so the trace can tell when the device passed it."""
        if not self._has_cuda:
            return None
        ev = NativeEvent(timing=self._trace_ref is not None)
        ev.record(_current_stream_handle())
        return ev

    def d2h_async(self, tensors: list[torch.Tensor],
                  after: "list[NativeEvent] | None" = None) -> tuple[list[torch.Tensor], "NativeEvent | SaveBackTicket | None"]:
        """Copies device tensors into new pinned host tensors (a save-back).

        Returns the host tensors and what marks their completion (None without a
        GPU, where the copies are synchronous). The device tensors are kept alive
        until the copies complete (``reap``/``drain``), so the caller may drop its
        references at once. Ordering: the copies start after the work queued so
        far on the current stream, or, given ``after``, once the device has passed
        every one of those events (the caller vouches that no work queued since
        writes the tensors).
        """
        if not self._has_cuda:
            return [t.detach().to("cpu").clone() for t in tensors], None
        outs, pairs = [], []
        for t in tensors:
            src = t.detach()
            if src.device.type == "cpu":
                outs.append(src.clone())
                continue
            if not src.is_contiguous():
                src = src.contiguous()
                after = None  # the contiguous copy is queued on the current stream now
            out = torch.empty(src.shape, dtype=src.dtype, pin_memory=True)
            outs.append(out)
            pairs.append((out, src))
        return outs, self._issue_save_back(pairs, "params", after)

    def d2h_into(self, src: torch.Tensor, dst: torch.Tensor,
                 after: "list[NativeEvent] | None" = None) -> "NativeEvent | SaveBackTicket | None":
        """One save-back copy of the contiguous device tensor ``src`` into the pinned host tensor
        ``dst``, after the work queued so far on the current stream (or after the events
        ``after``, as in ``d2h_async``); returns its completion."""
        nbytes = src.numel() * src.element_size()
        if dst.numel() * dst.element_size() < nbytes or not src.is_contiguous() or not dst.is_contiguous():
            raise ValueError("d2h_into needs contiguous tensors and a destination at least as large as the source")
        if not self._has_cuda:
            dst.view(torch.uint8)[:nbytes].copy_(src.reshape(-1).view(torch.uint8))
            return None
        return self._issue_save_back([(dst, src)], "block", after)

    def d2h_changed(self, src: torch.Tensor, dst: torch.Tensor, chunk: int, digests: torch.Tensor,
                    changed: torch.Tensor, after: "list[NativeEvent] | None" = None) -> "SaveBackTicket | None":
        """Save-back of the chunks of ``src`` (contiguous, on the device) whose digests differ from
        ``digests`` (written by a load's ``digest``) into ``dst`` (pinned host, which holds the bytes
        those digests describe), ordered as ``d2h_into``; ``changed`` is a pinned uint8 tensor of
        one byte per chunk. Returns None when this engine has no SDMA save-back engine (the caller
        then copies the whole tensor)."""
        sb = self._saveback_engine() if self._has_cuda else None
        if sb is None:
            return None
        nbytes = src.numel() * src.element_size()
        n_chunks = -(-nbytes // chunk)
        if (dst.numel() * dst.element_size() < nbytes or not src.is_contiguous() or not dst.is_contiguous()
                or changed.numel() < n_chunks or digests.numel() * digests.element_size() < 16 * n_chunks):
            raise ValueError("d2h_changed: buffers do not match the chunks")
        done = sb.submit_chunks([(dst.data_ptr(), src.data_ptr(), nbytes)], chunk, digests.data_ptr(),
                                changed.data_ptr(), self._loader_unpack_stream(), after, _current_stream_handle())
        keep = [dst, src, digests, changed]
        if after:
            keep.extend(after)
        if self._trace_ref is not None:
            fence = list(after) if after else None
            if fence is None:
                fence = [NativeEvent(timing=True)]
                fence[0].record(_current_stream_handle())
            self._trace_d2h.append((None, done, None, "block", fence, time.perf_counter()))
        self.bytes_d2h_requested += nbytes
        with self._lock:
            self._pending_d2h.append((done, keep, 0))
        return done

    def _saveback_engine(self) -> SaveBackEngine | None:
        """The SDMA save-back engine (created on first use), or None when save-backs use the copy stream."""
        if not self._has_cuda or self._save_back != "sdma":
            return None
        if self._saveback is None:
            try:
                self._saveback = SaveBackEngine(torch.cuda.current_device())
            except Exception as exc:  # noqa: BLE001 — the copy stream is the other device path
                log.warning("AsyncTransferEngine: no SDMA save-back engine (%s); save-backs use the copy stream", exc)
                self._save_back = "stream"
                return None
        return self._saveback

    def _issue_save_back(self, pairs: list[tuple[torch.Tensor, torch.Tensor]], kind: str,
                         after: "list[NativeEvent] | None" = None) -> "NativeEvent | SaveBackTicket":
        """Copies each (pinned host dst, device src) pair after the work queued so far on the current
        stream, or after the events ``after``: on the SDMA engine when there is one (one ticket),
        else on the copy stream (one event). Either way, completions are in submission order, and
        the pending list keeps the tensors alive until theirs."""
        nbytes = sum(src.numel() * src.element_size() for _dst, src in pairs)
        keep = [t for pair in pairs for t in pair]
        sb = self._saveback_engine()
        done: NativeEvent | SaveBackTicket
        if sb is not None:
            items = np.zeros(len(pairs), dtype=COPY_ITEM_DTYPE)
            for i, (dst, src) in enumerate(pairs):
                items[i] = (dst.data_ptr(), src.data_ptr(), src.numel() * src.element_size())
            if after:
                # the engine's worker waits for these events themselves (kept alive with the copy)
                done = sb.submit_after(items, after)
                keep.extend(after)
                fence = list(after)
            else:
                fence = None
                if self._trace_ref is not None:
                    # a timing event where the save-back's fence is recorded: when the device passes it
                    fence = [NativeEvent(timing=True)]
                    fence[0].record(_current_stream_handle())
                done = sb.submit(items, _current_stream_handle())
            if self._trace_ref is not None:
                self._trace_d2h.append((nbytes, done, None, kind, fence, time.perf_counter()))
        else:
            cs = self._copy_stream.cuda_stream
            if after:
                for ev in after:
                    ev.wait_on(cs)
            else:
                self._fence_copy_stream(cs)
            t_start = None
            if self._trace_ref is not None:
                t_start = NativeEvent(timing=True)
                t_start.record(cs)
            for dst, src in pairs:
                self._check_copy(_native.lib().sh_memcpy_d2h_async(dst.data_ptr(), src.data_ptr(),
                                                                   src.numel() * src.element_size(), cs), kind, "d2h")
            done = NativeEvent()
            done.record(cs)
            if t_start is not None:
                t_end = NativeEvent(timing=True)
                t_end.record(cs)
                self._trace_d2h.append((nbytes, t_start, t_end, kind))
        self.bytes_d2h += nbytes
        with self._lock:
            self._pending_d2h.append((done, keep, 0))
        return done

    def release_with_copy(self, ev: "NativeEvent | SaveBackTicket", nbytes: int) -> bool:
        """Counts ``nbytes`` of device memory as released from now on; the memory is freed when
        the save-back copy that ``ev`` completes is reaped (the copy holds it until then).

        The reference's save-back is synchronous, so its eviction loop sees the block's memory
        gone before it checks the low watermark again (src/stagehand/scheduler.py:1216-1226 and
        the loop at :1176-1182). Here the copy is still running, so the budget subtracts these
        bytes (:meth:`releasing_bytes`): otherwise one eviction round would evict every
        candidate. Returns False (nothing counted) when ``ev`` is not a save-back in flight.
        """
        if nbytes <= 0:
            return False
        with self._lock:
            for i in range(len(self._pending_d2h) - 1, -1, -1):
                e, keep, rel = self._pending_d2h[i]
                if e is ev:
                    self._pending_d2h[i] = (e, keep, rel + int(nbytes))
                    self._releasing_bytes += int(nbytes)
                    return True
        return False

    def releasing_bytes(self) -> int:
        """Device bytes given up with save-back copies that have not been reaped yet."""
        return self._releasing_bytes

    def wait_releasing(self, max_bytes: int) -> None:
        """Waits on the host for the oldest save-backs until at most ``max_bytes`` of released
        device memory is still held by copies in flight."""
        self._reap_d2h()
        while self._releasing_bytes > max_bytes:
            with self._lock:
                if not self._pending_d2h:
                    return
                ev = self._pending_d2h[0][0]
            with self.host_wait("save_back_backlog"):
                ev.synchronize()
            self._reap_d2h()

    def _reap_d2h(self, block: bool = False) -> None:
        """Drops the device references of completed save-back copies (they complete in order)."""
        while True:
            with self._lock:
                if not self._pending_d2h:
                    return
                ev = self._pending_d2h[0][0]
            if block:
                ev.synchronize()
            elif not ev.query():
                return
            with self._lock:
                if self._pending_d2h and self._pending_d2h[0][0] is ev:
                    self._releasing_bytes -= self._pending_d2h.pop(0)[2]
                else:
                    continue
            if getattr(ev, "counts_bytes", False):
                self.bytes_d2h += ev.copied_bytes()  # complete: returns at once

    # ── completion ───────────────────────────────────────────────────

    def poll(self, handle: TransferHandle) -> bool:
        if handle.completed:
            return True
        if handle.ticket is not None:
            st = _native.lib().sh_loader_query(self._loader, handle.ticket)
            if st == _native.SH_ERR_NOT_READY:
                return False
            if st != _native.SH_OK:
                self._raise_transfer(st, handle.block_id, handle.direction, handle)
            self._complete_handle(handle)
            return True
        if handle.event is None:
            if not self._has_cuda:
                return True
            return handle.completed
        done = handle.event.query()
        if done:
            self._complete_handle(handle)
        return done

    def wait_device(self, handle: TransferHandle, stream_handle: int | None = None) -> None:
        """Make ``stream_handle`` (default: current stream) wait for ``handle`` on the device."""
        if handle.completed or handle.device_waited:
            return
        if not self._has_cuda:
            self._complete_handle(handle)
            return
        sh = _current_stream_handle() if stream_handle is None else stream_handle
        if handle.ticket is not None:
            st = _native.lib().sh_loader_stream_wait(self._loader, handle.ticket, sh)
            if st != _native.SH_OK:
                self._raise_transfer(st, handle.block_id, handle.direction, handle)
        elif handle.event is not None:
            _native.call("sh_stream_wait_event", sh, handle.event.handle)
        handle.device_waited = True

    def wait(self, handle: TransferHandle) -> None:
        """Block the host until ``handle`` completes (the reference's wait), and order the current stream after it."""
        if handle.completed:
            return
        if handle.ticket is None and handle.event is None:
            self._complete_handle(handle)
            return
        t0 = time.monotonic()
        with self.host_wait("transfer_wait"):
            if handle.ticket is not None:
                st = _native.lib().sh_loader_sync(self._loader, handle.ticket)
                if st != _native.SH_OK:
                    self._raise_transfer(st, handle.block_id, handle.direction, handle)
            else:
                handle.event.synchronize()
        self.wait_device(handle)
        elapsed_ms = (time.monotonic() - t0) * 1000.0
        if _STALL_LOGS_ENABLED and elapsed_ms > 1.0:
            log.warning("Transfer stall: block=%s dir=%s wait=%.2f ms", handle.block_id, handle.direction, elapsed_ms)
        self._complete_handle(handle)

    def inflight_count(self) -> int:
        with self._lock:
            return len(self._inflight)

    def reap(self) -> int:
        self._reap_d2h()
        with self._lock:
            before = len(self._inflight)
            self._reap_completed_locked()
            return before - len(self._inflight)

    def drain(self) -> None:
        while True:
            with self._lock:
                remaining = list(self._inflight)
            if not remaining:
                break
            for h in remaining:
                self.wait(h)
        self._reap_d2h(block=True)

    def shutdown(self) -> None:
        try:
            self.drain()
            self.free_images()
        finally:
            if self._loader is not None:
                _native.call("sh_loader_destroy", self._loader)
                self._loader = None
            if self._saveback is not None:
                self._saveback.close()
                self._saveback = None
            if self._owned_stream is not None:
                _native.call("sh_stream_sync", self._owned_stream)
                _native.call("sh_stream_destroy", self._owned_stream)
                self._owned_stream = None

    def __del__(self) -> None:
        try:
            if self._loader is not None:
                _native.lib().sh_loader_destroy(self._loader)
                self._loader = None
        except Exception:
            pass

    # ── internals ────────────────────────────────────────────────────

    def _fence_copy_stream(self, copy_stream_handle: int) -> None:
        """The copy stream waits for work already queued on the current stream (e.g. the destination's allocation)."""
        ev = NativeEvent()
        ev.record(_current_stream_handle())
        _native.call("sh_stream_wait_event", copy_stream_handle, ev.handle)

    def _check_copy(self, status: int, block_id: str, direction: str) -> None:
        if status != _native.SH_OK:
            self._raise_transfer(status, block_id, direction)

    def _raise_transfer(self, status: int, block_id: str, direction: str,
                        handle: TransferHandle | None = None) -> None:
        msg = _native.last_error() or f"status {status}"
        if handle is not None:
            # a failed load is finished: later waits, drain() and shutdown() do not raise it again
            try:
                self._complete_handle(handle)
            except Exception:  # noqa: BLE001 — the original failure is the one to report
                pass
        if status == _native.SH_ERR_INVALID:
            raise ValueError(f"{direction} of block {block_id!r}: {msg}")
        raise TransferError(f"{direction} of block {block_id!r} failed: {msg}")

    def _make_handle(self, block_id: str, direction: str, size_bytes: int) -> TransferHandle:
        with self._lock:
            hid = self._next_handle_id
            self._next_handle_id += 1
        return TransferHandle(hid, block_id, direction, None, time.monotonic(), size_bytes)

    def _copy_outstanding(self, handle: TransferHandle) -> bool:
        """Whether ``handle``'s copy is still in flight. For a block load that is its H2D
        copies alone: its unpack and digests run where its first waiter queued them, possibly far
        ahead on a compute stream, and are not a transfer. A failed load holds no copy; its
        failure is raised where it is waited for. Called with the engine's lock held."""
        if handle.completed or handle.copy_landed:
            return False
        if handle.ticket is not None:
            st = _native.lib().sh_loader_query_copy(self._loader, handle.ticket)
            if st == _native.SH_ERR_NOT_READY:
                return True
            handle.copy_landed = True
            return False
        return True

    def _wait_for_slot(self) -> None:
        """Backpressure: block while ``max_inflight`` copies are outstanding.

        The reference polls in 1 ms condition waits (src/stagehand/transfer.py:258-276);
        here the host sleeps in a native wait on the oldest outstanding copy (copies on one
        stream complete in order), so a freed slot is seen at once. A wait above
        1 ms is logged at debug level: in a PCIe-bound stream it is the normal pacing.
        """
        self._reap_d2h()
        t0 = time.monotonic()
        while True:
            with self._cond:
                self._reap_completed_locked()
                outstanding = [h for h in self._inflight if self._copy_outstanding(h)]
                if len(outstanding) < self._max_inflight:
                    break
                oldest = outstanding[0]
            with self.host_wait("inflight_slot"):
                if oldest.ticket is not None:
                    st = _native.lib().sh_loader_sync_copy(self._loader, oldest.ticket)
                    if st != _native.SH_OK:
                        self._raise_transfer(st, oldest.block_id, oldest.direction)
                    oldest.copy_landed = True
                elif oldest.event is not None:
                    oldest.event.synchronize()
                else:
                    with self._cond:
                        self._cond.wait(timeout=0.001)
        waited_ms = (time.monotonic() - t0) * 1000.0
        if waited_ms > 1.0:
            log.debug("AsyncTransferEngine: backpressure wait %.2f ms", waited_ms)

    def _complete_handle(self, handle: TransferHandle) -> None:
        if handle.completed:
            return
        handle.completed = True
        if handle.ticket is not None and self._loader is not None:
            self._record_ticket_times(handle)
            _native.call("sh_loader_release", self._loader, handle.ticket)
            handle.ticket = None
        handle.keepalive = []
        with self._cond:
            try:
                self._inflight.remove(handle)
            except ValueError:
                pass
            self._cond.notify_all()

    def _reap_completed_locked(self) -> None:
        done: list[TransferHandle] = []
        for h in self._inflight:
            if h.completed:
                done.append(h)
            elif h.ticket is not None:
                st = _native.lib().sh_loader_query(self._loader, h.ticket)
                if st == _native.SH_OK:
                    done.append(h)
            elif h.event is not None and h.event.query():
                done.append(h)
            elif h.event is None and not self._has_cuda:
                done.append(h)
        for h in done:
            h.completed = True
            if h.ticket is not None and self._loader is not None:
                self._record_ticket_times(h)
                _native.lib().sh_loader_release(self._loader, h.ticket)
                h.ticket = None
            h.keepalive = []
            self._inflight.remove(h)
        if done:
            self._cond.notify_all()
