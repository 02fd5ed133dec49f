"""VMM residency backend: block weights in device virtual memory that is mapped
on demand and unmapped under a VRAM ceiling.

``SlabAllocator`` / ``ResidentHandle`` are the Python face of the reference's
pyo3 classes (vmm_src/python.rs:39-267) over the native allocator
(``sh_vmm_*`` in include/stagehand_native.h): same methods, arguments and
exception types (MemoryError when a region is watermarked or nothing can be
evicted, ValueError for a bad slab / region / dtype, RuntimeError for a
released handle or a slab with live handles). ``as_tensor`` exports the region
through DLPack with the ROCm device type; the tensor keeps its own reference to
the region.

``VmmModelHandle`` / ``VmmManager`` / ``is_available`` follow
src/stagehand/vmm_backend.py:21-440: one slab per model, one region per block,
weights populated on first use from a safetensors file or from host tensors.
Differences: regions start at granularity multiples (the reference places them
at running byte offsets); a block is re-populated whenever its region has been
re-mapped since it was filled (the reference's populate-once flag survives an
eviction, vmm_backend.py:205-208); the file is read through this package's
safetensors parser and ``mmap`` (the reference uses an external reader), and
with an ``AsyncTransferEngine`` the fill is a native block load (pinned
staging, copy stream) that the compute stream waits for on the device.
"""
from __future__ import annotations

import ctypes
import logging
import mmap
from pathlib import Path
from typing import Any, Optional

import numpy as np
import torch

from stagehand_amd import _native
from stagehand_amd._native import VMM_REGION_DTYPE, VMM_STATS_DTYPE

__all__ = ["SlabAllocator", "ResidentHandle", "VmmModelHandle", "VmmManager", "is_available", "RegionState"]

log = logging.getLogger(__name__)


class RegionState:
    UNMAPPED = 0
    MAPPED_EMPTY = 1
    RESIDENT = 2


# DLPack (code, bits) per dtype name (vmm_src/dlpack.rs:66-76); float8 is exported as
# uint8 bytes and viewed as float8 on the torch side.
_DL_DTYPES: dict[str, tuple[int, int, torch.dtype]] = {
    "float32": (2, 32, torch.float32),
    "float16": (2, 16, torch.float16),
    "bfloat16": (4, 16, torch.bfloat16),
    "int8": (0, 8, torch.int8),
    "int32": (0, 32, torch.int32),
    "int64": (0, 64, torch.int64),
    "uint8": (1, 8, torch.uint8),
    "float8_e4m3fn": (1, 8, torch.float8_e4m3fn),
}

_from_dlpack = torch._C._from_dlpack  # what torch.utils.dlpack.from_dlpack calls for a capsule
_fast_mod = None


def _fast():
    """The CPython binding of the hot path (``_lib/_sh_vmm``, built with the library): one C call
    for ensure_resident and one for the DLPack export, as the reference's pyo3 binding
    (vmm_src/python.rs:66-221). It links the library loaded by ``_native``."""
    global _fast_mod
    if _fast_mod is None:
        import importlib.util

        from stagehand_amd import build_native

        _native.lib()
        path = build_native.python_binding_path()
        if not path.exists():
            raise _native.NativeLibraryError(f"{path} is missing; build with python -m stagehand_amd.build_native")
        spec = importlib.util.spec_from_file_location("stagehand_amd._sh_vmm", str(path))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _fast_mod = mod
    return _fast_mod

_available: bool | None = None


def is_available() -> bool:
    """True when the native library is built and device 0 supports virtual memory management."""
    global _available
    if _available is not None:
        return _available
    try:
        if not torch.cuda.is_available():
            _available = False
            return False
        h = ctypes.c_void_p()
        st = _native.lib().sh_vmm_create(torch.cuda.current_device(), 0, ctypes.byref(h))
        if st == _native.SH_OK:
            _native.lib().sh_vmm_destroy(h)
        _available = st == _native.SH_OK
    except _native.NativeLibraryError:
        _available = False
    return _available


class SlabAllocator:
    """Native VMM allocator (vmm_src/python.rs:39-110)."""

    def __init__(self, device: int = 0, ceiling_mb: Optional[int] = None) -> None:
        h = ctypes.c_void_p()
        _native.call("sh_vmm_create", int(device), 0 if ceiling_mb is None else int(ceiling_mb) << 20, ctypes.byref(h))
        self._h = h
        self._hv: int | None = h.value  # the same pointer as a plain int, for the compiled binding
        self._ensure = _fast().ensure
        self._export = _fast().export
        self.device = int(device)
        _native.track(self, _native.CLOSE_ENGINE)

    def _handle(self) -> ctypes.c_void_p:
        if self._h is None:
            raise RuntimeError("VMM allocator has been closed")
        return self._h

    def create_slab(self, total_size: int) -> int:
        out = ctypes.c_uint32()
        _native.call("sh_vmm_create_slab", self._handle(), int(total_size), ctypes.byref(out))
        return out.value

    def define_region(self, slab: int, offset: int, size: int) -> int:
        out = ctypes.c_uint32()
        _native.call("sh_vmm_define_region", self._handle(), int(slab), int(offset), int(size), ctypes.byref(out))
        return out.value

    def ensure_resident(self, slab: int, region: int, stream: int) -> "ResidentHandle":
        """Maps the region if needed; ``stream`` is the consumer's stream handle
        (``torch.cuda.current_stream().cuda_stream``)."""
        h = self._hv
        if h is None:
            raise RuntimeError("VMM allocator has been closed")
        try:
            r = self._ensure(h, slab, region, stream)
        except TypeError:  # ids or stream given as another integer type (numpy, bool)
            r = self._ensure(h, int(slab), int(region), int(stream or 0))
        if r < 0:
            _native.check(-r, "sh_vmm_ensure_resident")
        handle = ResidentHandle.__new__(ResidentHandle)
        handle._h = r
        handle._alloc = self
        return handle

    def prefetch(self, slab: int, region: int) -> None:
        _native.call("sh_vmm_prefetch", self._handle(), int(slab), int(region))

    def time_fast_path(self, slab: int, region: int, stream: int, iters: int = 100_000) -> tuple[float, float]:
        """Native timing of ensure_resident on a resident region: (ns per call with the handles
        released after the loop, ns per call + release)."""
        out = (ctypes.c_double * 2)()
        _native.call("sh_vmm_time_fast_path", self._handle(), int(slab), int(region), int(stream), int(iters), out)
        return out[0], out[1]

    def set_priority(self, slab: int, priority: int) -> None:
        _native.call("sh_vmm_set_priority", self._handle(), int(slab), int(priority))

    def set_vram_ceiling(self, ceiling_bytes: int) -> None:
        _native.call("sh_vmm_set_ceiling", self._handle(), int(ceiling_bytes))

    def destroy_slab(self, slab: int) -> None:
        _native.call("sh_vmm_destroy_slab", self._handle(), int(slab))

    def stats(self) -> dict:
        st = np.zeros(1, dtype=VMM_STATS_DTYPE)
        _native.call("sh_vmm_info", self._handle(), st.ctypes.data)
        return {k: int(st[0][k]) for k in VMM_STATS_DTYPE.names}

    def granularity(self) -> int:
        return self.stats()["granularity"]

    def region_stats(self, slab: int, region: int) -> dict:
        st = np.zeros(1, dtype=VMM_REGION_DTYPE)
        _native.call("sh_vmm_region_info", self._handle(), int(slab), int(region), st.ctypes.data)
        return {k: int(st[0][k]) for k in VMM_REGION_DTYPE.names if k != "reserved"}

    def close(self) -> None:
        """Stops the prefetch worker; device memory goes once every handle is released."""
        if self._h is not None:
            _native.lib().sh_vmm_destroy(self._h)
            self._h = None
            self._hv = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


class ResidentHandle:
    """Keeps a region mapped while held (vmm_src/python.rs:111-267). ``_h`` is the native handle
    pointer as an int."""

    __slots__ = ("_h", "_alloc", "__weakref__")

    def __init__(self, handle: int, allocator: SlabAllocator) -> None:
        self._h = int(handle.value if isinstance(handle, ctypes.c_void_p) else handle)
        self._alloc = allocator  # keeps the Python allocator object alive while handles exist

    @property
    def released(self) -> bool:
        return self._h is None

    def data_ptr(self) -> int:
        if self._h is None:
            raise RuntimeError("Handle already released")
        out = ctypes.c_void_p()
        _native.call("sh_vmm_handle_ptr", self._h, ctypes.byref(out))
        return out.value

    def generation(self) -> int:
        """Mapping generation of the region: it changes at every (re)map, which loses the contents."""
        if self._h is None:
            raise RuntimeError("Handle already released")
        out = ctypes.c_uint64()
        _native.call("sh_vmm_handle_generation", self._h, ctypes.byref(out))
        return out.value

    def as_tensor(self, dtype: str, shape: list[int]) -> torch.Tensor:
        """A device tensor over the region (DLPack); it keeps the region mapped until it is freed."""
        h = self._h
        if h is None:
            raise RuntimeError("Handle already released")
        spec = _DL_DTYPES.get(dtype)
        if spec is None:
            raise ValueError(f"Unsupported dtype: {dtype}")
        code, bits, tdtype = spec
        cap = self._alloc._export(h, code, bits, shape)
        if type(cap) is int:
            _native.check(-cap, "sh_vmm_handle_export")
        t = _from_dlpack(cap)  # an unconsumed capsule frees its export when it is collected
        return t if t.dtype is tdtype else t.view(tdtype)

    def release(self) -> None:
        if self._h is None:
            raise RuntimeError("Handle already released")
        h, self._h = self._h, None
        _native.lib().sh_vmm_handle_destroy(h)

    def __del__(self) -> None:
        try:
            if self._h is not None:
                h, self._h = self._h, None
                _native.lib().sh_vmm_handle_destroy(h)
        except Exception:
            pass


# ── model handles (src/stagehand/vmm_backend.py:86-440) ──────────────────


class VmmModelHandle:
    """One slab per model, one region per block (vmm_backend.py:86-359)."""

    def __init__(self, allocator: SlabAllocator, model_id: str, block_sizes: list[int], dtype: str,
                 engine=None, file_reader: str = "mmap") -> None:
        if file_reader not in ("mmap", "pread", "direct"):
            raise ValueError(f"file_reader must be 'mmap', 'pread' or 'direct', got {file_reader!r}")
        self.allocator = allocator
        # "pread"/"direct": fills read the weight files with the native reader (file ranges
        # in the block load) instead of through mappings; needs the block loader
        self._file_reader = file_reader if engine is not None else "mmap"
        self.model_id = model_id
        self.dtype = dtype
        self.block_count = len(block_sizes)
        self.block_sizes = list(block_sizes)
        self._engine = engine
        gran = allocator.granularity()
        self._offsets = []
        offset = 0
        for size in block_sizes:
            self._offsets.append(offset)
            offset += -(-max(size, 1) // gran) * gran
        self.slab_id = allocator.create_slab(max(offset, gran))
        self.regions = [allocator.define_region(self.slab_id, off, max(size, 1))
                        for off, size in zip(self._offsets, block_sizes)]
        self.block_shapes: list[list[int] | None] = [None] * self.block_count
        self._active_handles: dict[int, ResidentHandle] = {}
        self._filled_generation: list[int | None] = [None] * self.block_count
        self._current_priority = 0
        self._destroyed = False
        self._files: dict[str, tuple] = {}  # path → (file object, mmap, memoryview)
        self._weight_files: dict[str, "WeightFile"] = {}  # path → native reader (file_reader != "mmap")
        # block → (handle, tensor, load, generation, stream) of a fill started ahead by prefetch_block
        self._pending_fills: dict[int, tuple] = {}
        self.fills_ahead = 0  # blocks served from a fill that prefetch_block started
        self._block_pieces: list[list[tuple[int, str, int, int]]] = []  # per block: (dst off, file, file off, bytes)
        self._ram_weight_refs: list[torch.Tensor | None] = [None] * self.block_count

    def register_block_shape(self, block_idx: int, shape: list[int]) -> None:
        self.block_shapes[block_idx] = list(shape)

    # ── weight sources ───────────────────────────────────────────────

    def set_mmap_source(self, safetensors_path: str, block_tensor_map: list[list[str]]) -> None:
        """Weights come from ``safetensors_path`` — one file, or a directory of shards with a
        ``*.safetensors.index.json`` — for each block, the named tensors back to back."""
        import json

        from stagehand_amd.registry import parse_safetensors_index

        src = Path(safetensors_path)
        where: dict[str, tuple[str, int, int]] = {}  # tensor → (file, offset, bytes)
        if src.is_dir():
            idx = next((src / n for n in ("diffusion_pytorch_model.safetensors.index.json",
                                          "model.safetensors.index.json") if (src / n).exists()), None)
            if idx is None:
                raise FileNotFoundError(f"No safetensors index found in {src}")
            for shard in dict.fromkeys(json.loads(idx.read_text())["weight_map"].values()):
                for k, meta in parse_safetensors_index(src / shard).items():
                    where[k] = (str(src / shard), meta[0], meta[1])
        else:
            for k, meta in parse_safetensors_index(src).items():
                where[k] = (str(src), meta[0], meta[1])
        pieces = []
        for names in block_tensor_map:
            dst, blk = 0, []
            for name in names:
                if name not in where:
                    raise KeyError(f"{name!r} is not in {safetensors_path}")
                path, off, nbytes = where[name]
                blk.append((dst, path, off, nbytes))
                dst += nbytes
            pieces.append(blk)
        self._close_file()
        for path in dict.fromkeys(p for blk in pieces for _d, p, _o, _n in blk):
            if self._file_reader != "mmap":
                from stagehand_amd.fileio import WeightFile

                self._weight_files[path] = WeightFile(path, direct=self._file_reader == "direct")
                continue
            fh = open(path, "rb")
            mm = mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ)
            self._files[path] = (fh, mm, memoryview(mm))
        self._block_pieces = pieces
        self._filled_generation = [None] * self.block_count

    def set_ram_weights(self, block_idx: int, weights: torch.Tensor) -> None:
        self._ram_weight_refs[block_idx] = weights

    def _close_file(self) -> None:
        for fh, mm, view in self._files.values():
            for fn in (view.release, mm.close, fh.close):
                try:
                    fn()
                except Exception:
                    pass
        self._files = {}
        if self._weight_files and self._engine is not None:
            self._engine.drain()  # queued loads may still read the files
        for wf in self._weight_files.values():
            wf.close()
        self._weight_files = {}

    # ── block access ─────────────────────────────────────────────────

    def get_block_tensor(self, block_idx: int, stream: int) -> tuple[torch.Tensor | None, bool]:
        """(tensor, True), or (None, False) when the region is watermarked (vmm_backend.py:190-222)."""
        if self.block_shapes[block_idx] is None:
            raise RuntimeError(f"Block {block_idx} shape not registered. Call register_block_shape first.")
        pending = self._pending_fills.pop(block_idx, None)
        if pending is not None:
            # filled ahead by prefetch_block: the caller's stream waits for that load on the device
            p_handle, tensor, load, gen, p_stream = pending
            if p_stream != stream:
                # a handle's release orders eviction after its own stream: take one on the caller's
                # (the region is held throughout, so the fill cannot be unmapped under the load)
                own = self.allocator.ensure_resident(self.slab_id, self.regions[block_idx], stream)
                p_handle.release()
                p_handle = own
            self._engine.wait_device(load, stream)
            self._filled_generation[block_idx] = gen
            self._active_handles[block_idx] = p_handle
            self.fills_ahead += 1
            return tensor, True
        handle = None
        try:
            handle = self.allocator.ensure_resident(self.slab_id, self.regions[block_idx], stream)
            tensor = handle.as_tensor(self.dtype, self.block_shapes[block_idx])
            gen = handle.generation()
            if self._filled_generation[block_idx] != gen:
                self._populate_block(block_idx, tensor)
                self._filled_generation[block_idx] = gen
            self._active_handles[block_idx] = handle
            return tensor, True
        except MemoryError:
            if handle is not None:
                handle.release()
            return None, False
        except Exception:
            if handle is not None and not handle.released:
                handle.release()
            raise

    def _host_pieces(self, block_idx: int) -> list[tuple[int, Any]]:
        if self._weight_files and block_idx < len(self._block_pieces):
            from stagehand_amd.fileio import FileRange

            return [(dst, FileRange(self._weight_files[path], off, n))
                    for dst, path, off, n in self._block_pieces[block_idx] if n > 0]
        if self._files and block_idx < len(self._block_pieces):
            return [(dst, torch.frombuffer(self._files[path][2], dtype=torch.uint8, count=n, offset=off))
                    for dst, path, off, n in self._block_pieces[block_idx] if n > 0]
        ram = self._ram_weight_refs[block_idx]
        if ram is not None:
            return [(0, ram.detach().reshape(-1).contiguous().view(torch.uint8))]
        raise RuntimeError(f"No weight source for block {block_idx}")

    def _submit_fill(self, block_idx: int, vmm_tensor: torch.Tensor):
        """Starts the load of the block's weights into its region; returns the transfer handle."""
        from stagehand_amd.transfer import BlockSource

        dst = vmm_tensor.view(-1).view(torch.uint8)
        pieces = self._host_pieces(block_idx)
        src_bytes = max((off + t.numel() for off, t in pieces), default=0)
        return self._engine.submit_block_load(f"{self.model_id}:{block_idx}", BlockSource(pieces, src_bytes),
                                              dst[:src_bytes])

    def _populate_block(self, block_idx: int, vmm_tensor: torch.Tensor) -> None:
        dst = vmm_tensor.view(-1).view(torch.uint8)
        pieces = self._host_pieces(block_idx)
        if self._engine is not None and torch.cuda.is_available():
            self._engine.wait_device(self._submit_fill(block_idx, vmm_tensor))
        else:
            for off, t in pieces:
                dst[off:off + t.numel()].copy_(t, non_blocking=True)

    def fits_without_eviction(self, block_idx: int) -> bool:
        """True when the block's region fits beside everything mapped now, under the ceiling."""
        if not 0 <= block_idx < self.block_count:
            return False
        st = self.allocator.stats()
        g = max(1, int(st["granularity"]))
        need = -(-int(self.block_sizes[block_idx]) // g) * g
        return int(st["mapped_bytes"]) + need <= int(st["vram_ceiling"])

    def prefetch_block(self, block_idx: int, stream: int | None = None) -> None:
        """Maps the block's region ahead and warms its file pages (vmm_backend.py:283-291). With the
        block loader and a ``stream``, a region whose contents are stale is mapped now and its fill
        starts on the loader at once, holding the region until ``get_block_tensor`` takes it."""
        if not 0 <= block_idx < self.block_count:
            return
        if (stream is not None and self._engine is not None and torch.cuda.is_available()
                and self.block_shapes[block_idx] is not None and block_idx not in self._pending_fills
                and block_idx not in self._active_handles):
            handle = None
            try:
                handle = self.allocator.ensure_resident(self.slab_id, self.regions[block_idx], stream)
                gen = handle.generation()
                if self._filled_generation[block_idx] == gen:
                    handle.release()  # mapped and filled already
                    return
                tensor = handle.as_tensor(self.dtype, self.block_shapes[block_idx])
                load = self._submit_fill(block_idx, tensor)
                self._pending_fills[block_idx] = (handle, tensor, load, gen, stream)
                return
            except MemoryError:
                if handle is not None and not handle.released:
                    handle.release()
            except Exception:
                if handle is not None and not handle.released:
                    handle.release()
                raise
        try:
            self.allocator.prefetch(self.slab_id, self.regions[block_idx])
        except Exception:
            pass
        if self._weight_files and block_idx < len(self._block_pieces):
            for _dst, path, off, n in self._block_pieces[block_idx]:
                try:
                    self._weight_files[path].advise_willneed(off, n)
                except OSError:
                    pass
        if self._files and block_idx < len(self._block_pieces):
            page = mmap.PAGESIZE
            for _dst, path, off, n in self._block_pieces[block_idx]:
                start = off // page * page
                try:
                    self._files[path][1].madvise(mmap.MADV_WILLNEED, start, off + n - start)
                except (AttributeError, OSError, ValueError):
                    pass

    # ── lifecycle ────────────────────────────────────────────────────

    def release_block(self, block_idx: int) -> None:
        handle = self._active_handles.pop(block_idx, None)
        if handle is not None and not handle.released:
            handle.release()

    def set_priority(self, priority: int) -> None:
        self._current_priority = priority
        self.allocator.set_priority(self.slab_id, priority)

    def invalidate_weights(self) -> None:
        self._filled_generation = [None] * self.block_count

    def release_all(self) -> None:
        for idx in list(self._active_handles):
            self.release_block(idx)
        self._drop_pending_fills()

    def _drop_pending_fills(self) -> None:
        """Releases fills started ahead and never taken, after their loads on the device (a
        region's release orders its eviction after the work on the handle's stream)."""
        for _idx, (handle, _tensor, load, _gen, stream) in list(self._pending_fills.items()):
            self._engine.wait_device(load, stream)
            if not handle.released:
                handle.release()
        self._pending_fills.clear()

    def release_mmap(self) -> None:
        """Lets the OS drop the file's pages (they are re-read on the next fill)."""
        for _fh, mm, _view in self._files.values():
            try:
                mm.madvise(mmap.MADV_DONTNEED)
            except (AttributeError, OSError):
                pass

    def destroy(self) -> None:
        if self._destroyed:
            return
        self._destroyed = True
        self.release_all()
        self._ram_weight_refs = [None] * self.block_count
        if torch.cuda.is_available():
            torch.cuda.synchronize()  # fills may still read the file's pages
        if self._engine is not None:
            self._engine.drain()
        self._close_file()
        try:
            self.allocator.destroy_slab(self.slab_id)
        except Exception as e:
            log.warning("VMM: destroy_slab failed for %s: %s", self.model_id, e)

    def __del__(self) -> None:
        if self._destroyed:
            return
        if self._active_handles:
            log.warning("VMM: %s dropped with %d active handles; slab kept", self.model_id, len(self._active_handles))
            return
        try:
            self.destroy()
        except Exception:
            pass


class VmmManager:
    """The allocator and its per-model handles (vmm_backend.py:365-440)."""

    def __init__(self, device: int = 0, ceiling_mb: Optional[int] = None, engine=None,
                 file_reader: str = "mmap") -> None:
        if not is_available():
            raise RuntimeError("VMM backend not available")
        self.allocator = SlabAllocator(device=device, ceiling_mb=ceiling_mb)
        self.models: dict[str, VmmModelHandle] = {}
        self._priority_counter = 0
        self._engine = engine
        self._file_reader = file_reader
        _native.track(self, _native.CLOSE_ENGINE_USER, "shutdown")
        s = self.allocator.stats()
        log.info("VMM: allocator ready. ceiling=%.2fGB, granularity=%.1fMB", s["vram_ceiling"] / 1e9,
                 s["granularity"] / 1e6)

    def register_model(self, model_id: str, block_sizes: list[int], dtype: str) -> VmmModelHandle:
        if model_id in self.models:
            log.warning("VMM: %s already registered, replacing", model_id)
            self.models[model_id].destroy()
        handle = VmmModelHandle(self.allocator, model_id, block_sizes, dtype, engine=self._engine,
                                file_reader=self._file_reader)
        self.models[model_id] = handle
        return handle

    def activate_model(self, model_id: str) -> None:
        if model_id not in self.models:
            return
        self._priority_counter += 1
        self.models[model_id].set_priority(self._priority_counter)
        for mid, handle in self.models.items():
            if mid != model_id:
                handle.release_mmap()

    def unregister_model(self, model_id: str) -> None:
        handle = self.models.pop(model_id, None)
        if handle is not None:
            handle.destroy()

    def set_ceiling(self, ceiling_bytes: int) -> None:
        self.allocator.set_vram_ceiling(ceiling_bytes)

    def stats(self) -> dict:
        s = self.allocator.stats()
        mm = sum(len(f[1]) for h in self.models.values() for f in h._files.values())
        s["mmap_data_bytes"] = mm
        s["mmap_data_gb"] = round(mm / 1e9, 2)
        return s

    def shutdown(self) -> None:
        for mid in list(self.models):
            self.unregister_model(mid)
        self.allocator.close()
