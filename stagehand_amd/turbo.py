"""Turbo window engine: blocks rotate through a fixed window of device slots.

``TransferEngine`` is the Python face of the reference's pyo3 class
(turbo_src/lib.rs:14-126) over the native engine in
``stagehand_amd/csrc/sh_turbo.cpp``: the same methods, arguments, return
values and exception types. ``step`` takes an optional stream (the caller's
compute stream; the torch current stream by default) because the engine
orders compute after a block's copy on the device instead of blocking the
host. Extra methods: ``set_slot_buffer`` / ``slot_bytes`` /
``param_offset`` (a slot as one contiguous buffer, a block in one copy),
``set_writeback`` (no D2H for frozen blocks), ``set_save_back`` (write-backs on
an SDMA engine or the evict stream) and ``bytes_moved``.

``TurboConductor`` keeps the reference's conductor interface
(src/stagehand/turbo.py:29-201): discover blocks by pattern, ``prepare`` them
(pinned host copies of every block, a window of 3 slots), ``before_block`` /
``after_block`` around each block's compute, ``evict_all``, ``shutdown``.
Its slots are contiguous device buffers, and blocks whose parameters are all
frozen are not copied back at eviction.
"""
from __future__ import annotations

import ctypes
import logging
import re

import numpy as np
import torch
from torch import nn

from stagehand_amd import _native

__all__ = ["TransferEngine", "TurboConductor", "is_available"]

log = logging.getLogger(__name__)

_LOCATIONS = {0: "cpu", 1: "gpu", 2: "h2d", 3: "d2h"}
_DIRECTIONS = {"forward": 0, "backward": 1}


def is_available() -> bool:
    """True when the native library is built (the engine needs nothing else)."""
    try:
        _native.lib()
        return True
    except _native.NativeLibraryError:
        return False


def _stream_handle(stream) -> int:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream if torch.cuda.is_available() else 0
    return stream if isinstance(stream, int) else stream.cuda_stream


class TransferEngine:
    """Window engine with the reference's pyo3 API (turbo_src/lib.rs:14-126)."""

    def __init__(self) -> None:
        h = ctypes.c_void_p()
        _native.call("sh_turbo_create", ctypes.byref(h))
        self._h = h
        _native.track(self, _native.CLOSE_ENGINE)

    def _handle(self) -> ctypes.c_void_p:
        if self._h is None:
            raise RuntimeError("turbo engine has been closed")
        return self._h

    def register_block(self, param_sizes: list[int]) -> int:
        sizes = np.ascontiguousarray(param_sizes, dtype=np.uint64)
        if sizes.size and int(sizes.min()) < 0:
            raise OverflowError("param sizes must be non-negative")
        idx = ctypes.c_uint32()
        _native.call("sh_turbo_register_block", self._handle(), sizes.ctypes.data, sizes.size, ctypes.byref(idx))
        return idx.value

    def set_save_back(self, engine: str) -> None:
        """Before ``initialize``: write-backs on an SDMA engine ("sdma", the default) or as
        ``hipMemcpyAsync`` on the engine's evict stream ("stream")."""
        if engine not in ("sdma", "stream"):
            raise ValueError(f"save_back must be 'sdma' or 'stream', got {engine!r}")
        _native.call("sh_turbo_set_save_back", self._handle(), int(engine == "sdma"))

    def set_writeback_chunks(self, chunk_bytes: int) -> None:
        """Before ``initialize``: SDMA write-backs copy only the chunks of ``chunk_bytes`` (default
        256 KiB) that changed in the slot since the block's H2D (chunk digests on the device); 0
        copies every byte, as the reference does (turbo_src/engine.rs:232-262). The host region
        ends up the same either way."""
        _native.call("sh_turbo_set_writeback_chunks", self._handle(), int(chunk_bytes))

    def initialize(self, device: int, window_size: int) -> None:
        _native.call("sh_turbo_initialize", self._handle(), int(device), int(window_size))

    def stage_block(self, block_idx: int, src_ptrs: list[int]) -> None:
        arr = np.ascontiguousarray(src_ptrs, dtype=np.uint64)
        _native.call("sh_turbo_stage_block", self._handle(), int(block_idx), arr.ctypes.data, arr.size)

    def step(self, block_idx: int, direction: str, stream=None) -> None:
        if direction not in _DIRECTIONS:
            raise ValueError("direction must be 'forward' or 'backward'")
        _native.call("sh_turbo_step", self._handle(), int(block_idx), _DIRECTIONS[direction], _stream_handle(stream))

    def evict_sync(self, block_idx: int, stream=None) -> None:
        _native.call("sh_turbo_evict_sync", self._handle(), int(block_idx), _stream_handle(stream))

    def gpu_ptr(self, block_idx: int, param_idx: int) -> int:
        out = ctypes.c_uint64()
        _native.call("sh_turbo_gpu_ptr", self._handle(), int(block_idx), int(param_idx), ctypes.byref(out))
        return out.value

    def cpu_ptr(self, block_idx: int, param_idx: int) -> int:
        out = ctypes.c_uint64()
        _native.call("sh_turbo_cpu_ptr", self._handle(), int(block_idx), int(param_idx), ctypes.byref(out))
        return out.value

    def param_offset(self, block_idx: int, param_idx: int) -> int:
        out = ctypes.c_uint64()
        _native.call("sh_turbo_param_offset", self._handle(), int(block_idx), int(param_idx), ctypes.byref(out))
        return out.value

    def set_slot_gpu_ptrs(self, slot_idx: int, ptrs: list[int]) -> None:
        arr = np.ascontiguousarray(ptrs, dtype=np.uint64)
        _native.call("sh_turbo_set_slot_gpu_ptrs", self._handle(), int(slot_idx), arr.ctypes.data, arr.size)

    def set_slot_buffer(self, slot_idx: int, base_ptr: int, nbytes: int) -> None:
        _native.call("sh_turbo_set_slot_buffer", self._handle(), int(slot_idx), int(base_ptr), int(nbytes))

    def slot_bytes(self) -> int:
        out = ctypes.c_uint64()
        _native.call("sh_turbo_slot_bytes", self._handle(), ctypes.byref(out))
        return out.value

    def set_writeback(self, block_idx: int, enabled: bool) -> None:
        _native.call("sh_turbo_set_writeback", self._handle(), int(block_idx), int(bool(enabled)))

    def block_slot(self, block_idx: int) -> int | None:
        out = ctypes.c_int32()
        _native.call("sh_turbo_block_slot", self._handle(), int(block_idx), ctypes.byref(out))
        return None if out.value < 0 else out.value

    def _counts(self) -> tuple[int, int, int]:
        b, s, f = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint32()
        _native.call("sh_turbo_counts", self._handle(), ctypes.byref(b), ctypes.byref(s), ctypes.byref(f))
        return b.value, s.value, f.value

    def num_blocks(self) -> int:
        return self._counts()[0]

    def num_gpu_slots(self) -> int:
        return self._counts()[1]

    def num_free_slots(self) -> int:
        return self._counts()[2]

    def block_location(self, block_idx: int) -> str:
        out = ctypes.c_int()
        _native.call("sh_turbo_block_location", self._handle(), int(block_idx), ctypes.byref(out))
        return _LOCATIONS[out.value]

    def bytes_moved(self) -> tuple[int, int]:
        h2d, d2h = ctypes.c_uint64(), ctypes.c_uint64()
        _native.call("sh_turbo_bytes", self._handle(), ctypes.byref(h2d), ctypes.byref(d2h))
        return h2d.value, d2h.value

    def set_timing(self, enabled: bool) -> None:
        _native.call("sh_turbo_set_timing", self._handle(), int(bool(enabled)))

    def block_times(self, block_idx: int, ref_event) -> tuple[float, float]:
        """Start and end (ms after ``ref_event``, a native timing event) of the block's last H2D."""
        out = (ctypes.c_float * 2)()
        _native.call("sh_turbo_block_times", self._handle(), int(block_idx), ref_event.handle, out)
        return out[0], out[1]

    def trace_spans(self):
        """Write-back and host-wait spans recorded since timing was switched on (a numpy array
        of ``_native.TURBO_SPAN_DTYPE``, times on the save-back engine's HSA clock)."""
        n = ctypes.c_uint32()
        _native.call("sh_turbo_trace_spans", self._handle(), None, 0, ctypes.byref(n))
        out = np.zeros(n.value, dtype=_native.TURBO_SPAN_DTYPE)
        if n.value:
            _native.call("sh_turbo_trace_spans", self._handle(), out.ctypes.data, n.value, ctypes.byref(n))
        return out[:n.value]

    def drain(self) -> None:
        _native.call("sh_turbo_drain", self._handle())

    def close(self) -> None:
        if self._h is not None:
            _native.lib().sh_turbo_destroy(self._h)
            self._h = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


class TurboConductor:
    """Block-swap conductor over the window engine (src/stagehand/turbo.py:29-201)."""

    WINDOW = 3  # slots, as src/stagehand/turbo.py:98-100

    def __init__(self, model: nn.Module, block_pattern: str = r".*\.block\.\d+$", dtype: torch.dtype = torch.bfloat16,
                 device: int = 0, vram_budget_gb: float = 18.0, *, contiguous_slots: bool = True,
                 writeback: str = "auto", save_back: str = "sdma", window: int | None = None,
                 writeback_chunk_bytes: int = 1 << 18) -> None:
        """``contiguous_slots=False`` gives every parameter position its own slot tensor, as
        src/stagehand/turbo.py:123-147 does (one copy per parameter); ``writeback`` is
        "auto" (copy back only blocks with trainable parameters) or "always" (as
        turbo_src/engine.rs:233-264 does); ``save_back`` is where write-backs run
        (``TransferEngine.set_save_back``); ``window`` is the number of device slots (default
        ``WINDOW``, the reference's 3, at least 3). With write-back, every prefetch into a slot
        waits for the write-back out of it; more slots give it more time. SDMA write-backs copy
        only the chunks of ``writeback_chunk_bytes`` that changed on the device (0: every byte;
        ``TransferEngine.set_writeback_chunks``)."""
        _native.lib()  # fail loudly without the native library
        if writeback not in ("auto", "always"):
            raise ValueError(f"writeback must be 'auto' or 'always', got {writeback!r}")
        if save_back not in ("sdma", "stream"):
            raise ValueError(f"save_back must be 'sdma' or 'stream', got {save_back!r}")
        self._save_back = save_back
        self._writeback_chunk_bytes = int(writeback_chunk_bytes)
        self._window = self.WINDOW if window is None else int(window)
        if self._window < 3:
            # a step loads its block before it evicts the previous one, and the last block of a
            # pass keeps its slot into the next pass (engine.rs:304-341)
            raise ValueError(f"window must be at least 3, got {window!r}")
        self._contiguous = contiguous_slots
        self._writeback = writeback
        self._dtype = dtype
        self._device_idx = device
        self._device = torch.device(f"cuda:{device}")
        self._vram_budget_gb = vram_budget_gb
        pat = re.compile(block_pattern)
        self._block_names: list[str] = []
        self._block_modules: list[nn.Module] = []
        for name, mod in model.named_modules():
            if pat.match(name):
                self._block_names.append(name)
                self._block_modules.append(mod)
        if not self._block_modules:
            raise ValueError(f"No blocks matched {block_pattern!r}")
        self._engine: TransferEngine | None = None
        self._prepared = False
        self._param_meta: list[list[tuple[str, tuple[int, ...], int]]] = []
        self._slot_tensors: list = []  # contiguous: one uint8 tensor per slot; else a list per slot
        self._cpu_tensors: list[list[torch.Tensor]] = []
        self._offsets: list[list[int]] = []
        self._trace_ref = None
        self._trace_t0_ns = 0
        self._trace_compute: list = []
        self._trace_loaded: list[int] = []
        log.info("TurboConductor: %d blocks", len(self._block_modules))

    @property
    def num_blocks(self) -> int:
        return len(self._block_modules)

    @property
    def engine(self) -> TransferEngine | None:
        return self._engine

    def prepare(self) -> None:
        if self._prepared:
            return
        engine = TransferEngine()
        for mod in self._block_modules:
            meta = [(n, tuple(p.shape), p.numel() * self._dtype.itemsize) for n, p in mod.named_parameters()]
            engine.register_block([m[2] for m in meta])
            self._param_meta.append(meta)
        engine.set_save_back(self._save_back)
        engine.set_writeback_chunks(self._writeback_chunk_bytes)
        engine.initialize(self._device_idx, self._window)
        for bi, mod in enumerate(self._block_modules):
            params = list(mod.named_parameters())
            src = [p.data.detach().to("cpu", self._dtype).contiguous() for _n, p in params]
            engine.stage_block(bi, [t.data_ptr() if t.numel() else 0 for t in src])
            del src
            # frozen blocks are never written on the device: nothing to copy back
            engine.set_writeback(bi, self._writeback == "always" or any(p.requires_grad for _n, p in params))
            views, offs = [], []
            for pi, (_n, shape, nbytes) in enumerate(self._param_meta[bi]):
                offs.append(engine.param_offset(bi, pi))
                if nbytes == 0:
                    views.append(torch.empty(shape, dtype=self._dtype))
                    continue
                buf = (ctypes.c_char * nbytes).from_address(engine.cpu_ptr(bi, pi))
                views.append(torch.frombuffer(buf, dtype=self._dtype).reshape(shape))
            self._cpu_tensors.append(views)
            self._offsets.append(offs)
        slot_bytes = engine.slot_bytes()
        n_pos = max(len(m) for m in self._param_meta)
        cap = [max((m[p][2] for m in self._param_meta if p < len(m)), default=0) for p in range(n_pos)]
        for si in range(engine.num_gpu_slots()):
            if self._contiguous:
                t = torch.empty(max(slot_bytes, 1), dtype=torch.uint8, device=self._device)
                engine.set_slot_buffer(si, t.data_ptr(), t.numel())
                self._slot_tensors.append(t)
            else:
                ts = [torch.empty(max(c, 1), dtype=torch.uint8, device=self._device) for c in cap]
                engine.set_slot_gpu_ptrs(si, [t.data_ptr() for t in ts])
                self._slot_tensors.append(ts)
        for bi, mod in enumerate(self._block_modules):
            for pi, (_n, p) in enumerate(mod.named_parameters()):
                p.data = self._cpu_tensors[bi][pi]
        self._engine = engine
        self._prepared = True
        log.info("TurboConductor: ready, %d slots of %d bytes, %d blocks", len(self._slot_tensors), slot_bytes,
                 len(self._block_modules))

    def before_block(self, block_idx: int, direction: str = "forward") -> None:
        """Make the block resident and point its parameters at its slot (device-side ordering)."""
        assert self._engine is not None
        if self._trace_ref is not None:
            self._trace_step_loads(block_idx, direction)
        self._engine.step(block_idx, direction)
        if self._trace_ref is not None:
            self._trace_mark(block_idx, True)
        slot = self._engine.block_slot(block_idx)
        if slot is None:
            raise RuntimeError(f"Block {block_idx} has no GPU slot after step()")
        held = self._slot_tensors[slot]
        for pi, (_n, p) in enumerate(self._block_modules[block_idx].named_parameters()):
            _name, shape, nbytes = self._param_meta[block_idx][pi]
            if self._contiguous:
                off = self._offsets[block_idx][pi]
                p.data = held[off:off + nbytes].view(self._dtype).view(shape)
            else:
                p.data = held[pi][:nbytes].view(self._dtype).view(shape)

    def after_block(self, block_idx: int) -> None:
        if self._trace_ref is not None:
            self._trace_mark(block_idx, False)
        for pi, (_n, p) in enumerate(self._block_modules[block_idx].named_parameters()):
            p.data = self._cpu_tensors[block_idx][pi]

    def evict_all(self) -> None:
        if self._engine is None:
            return
        for idx in range(len(self._block_modules)):
            if self._engine.block_location(idx) in ("gpu", "h2d"):
                self._engine.evict_sync(idx)
        for bi, mod in enumerate(self._block_modules):
            for pi, (_n, p) in enumerate(mod.named_parameters()):
                p.data = self._cpu_tensors[bi][pi]

    # ── device timeline (not in the reference) ───────────────────────

    def start_trace(self) -> None:
        """Time every later block H2D and the compute between before_block and after_block,
        relative to an event recorded now on the current stream."""
        from stagehand_amd.transfer import NativeEvent, SaveBackEngine

        assert self._engine is not None
        self._engine.set_timing(True)
        self._trace_ref = NativeEvent(timing=True)
        self._trace_ref.record(torch.cuda.current_stream().cuda_stream)
        # write-back and host-wait spans are on the HSA clock: read it when the reference event completes
        self._trace_ref.synchronize()
        self._trace_t0_ns = SaveBackEngine.clock_ns()
        self._trace_compute, self._trace_loaded = [], []

    def _trace_step_loads(self, block_idx: int, direction: str) -> None:
        # blocks whose H2D this step() issues: the block itself (if not resident) and the lookahead
        n = len(self._block_modules)
        nxt = block_idx + 1 if direction == "forward" else block_idx - 1
        for b in (block_idx, nxt):
            if 0 <= b < n and self._engine.block_location(b) in ("cpu", "d2h"):
                self._trace_loaded.append(b)

    def _trace_mark(self, block_idx: int, start: bool) -> None:
        from stagehand_amd.transfer import NativeEvent

        ev = NativeEvent(timing=True)
        ev.record(torch.cuda.current_stream().cuda_stream)
        if start:
            self._trace_compute.append([block_idx, ev, None])
        else:
            for rec in reversed(self._trace_compute):
                if rec[0] == block_idx and rec[2] is None:
                    rec[2] = ev
                    break

    def stop_trace(self) -> dict:
        """{"loads": [(block, bytes, start, end, end)], "compute": [(block, start, end)],
        "d2h": [(bytes, start, end, "writeback")], "host_waits": [("slot_reuse", start, end)]}, in ms
        after start_trace; "d2h_untimed" counts write-backs without copy times."""
        if self._trace_ref is None:
            return {"loads": [], "compute": []}
        torch.cuda.synchronize()
        ref = self._trace_ref
        loads = []
        for b in dict.fromkeys(self._trace_loaded):
            t0, t1 = self._engine.block_times(b, ref)
            loads.append((self._block_names[b], sum(m[2] for m in self._param_meta[b]), t0, t1, t1))
        compute = [(self._block_names[b], ref.elapsed_ms(s), ref.elapsed_ms(e)) for b, s, e in self._trace_compute
                   if e is not None]
        d2h, waits, untimed = [], [], 0
        t0_ns = self._trace_t0_ns
        for sp in self._engine.trace_spans():
            start, end = (int(sp["start_ns"]) - t0_ns) / 1e6, (int(sp["end_ns"]) - t0_ns) / 1e6
            if sp["kind"] == _native.TURBO_SPAN_HOST_WAIT:
                waits.append(("slot_reuse", start, end))
            elif sp["bytes"] == 0:
                continue  # a write-back of changed chunks that found none: no copy
            elif sp["start_ns"] == 0:
                untimed += 1
            else:
                d2h.append((int(sp["bytes"]), start, end, "writeback"))
        self._engine.set_timing(False)
        self._trace_ref = None
        self._trace_compute, self._trace_loaded = [], []
        return {"loads": loads, "compute": compute, "d2h": d2h, "d2h_untimed": untimed, "host_waits": waits}

    def install_hooks(self) -> list:
        """Forward pre/post hooks that call before_block / after_block (not in the reference)."""
        handles = []
        for i, mod in enumerate(self._block_modules):
            handles.append(mod.register_forward_pre_hook(lambda _m, _a, i=i: self.before_block(i, "forward")))
            handles.append(mod.register_forward_hook(lambda _m, _a, _o, i=i: self.after_block(i)))
        return handles

    def shutdown(self, restore_params: bool = True) -> None:
        """Drain and free the engine. The parameters point at the engine's pinned
        memory between blocks, so with ``restore_params`` they get host copies of
        their own first (else they are left empty)."""
        if self._engine is not None:
            self._engine.drain()
            for bi, mod in enumerate(self._block_modules):
                for pi, (_n, p) in enumerate(mod.named_parameters()):
                    view = self._cpu_tensors[bi][pi]
                    p.data = view.clone() if restore_params else view.new_empty(0)
        self._slot_tensors.clear()
        self._cpu_tensors.clear()
        if self._engine is not None:
            self._engine.close()
            self._engine = None
