"""Fixed pinned host slab pool with backpressure (native).

Same Python contract as src/stagehand/pool.py:42-246 — ``PinnedPool(total_mb,
slab_mb, alignment)``, ``acquire(size) -> PinnedSlab | list[PinnedSlab]``,
``release``, ``stats``, ``shutdown``, ``slab_bytes``, ``num_slabs``; a
``PinnedSlab`` has ``slab_id``, ``buffer`` (uint8 tensor), ``size_bytes``,
``pool_id`` — over the native pool of ``include/stagehand_native.h``: one
hipHostMalloc region cut into slabs, acquire blocking in native code with the
GIL released. ``release_after(slab, stream)`` additionally returns a slab only
once the copies queued on ``stream`` have drained, without blocking the host.
Without a GPU the memory is ordinary host memory, as in the reference.
"""
from __future__ import annotations

import ctypes
import logging
import math
from dataclasses import dataclass

import numpy as np
import torch

from stagehand_amd import _native
from stagehand_amd._native import POOL_STATS_DTYPE
from stagehand_amd.errors import StagehandOOMError

__all__ = ["PinnedPool", "PinnedSlab"]

log = logging.getLogger(__name__)

_WARN_MS = 100.0


@dataclass
class PinnedSlab:
    slab_id: int
    buffer: torch.Tensor
    size_bytes: int
    pool_id: int

    def data_ptr(self) -> int:
        return self.buffer.data_ptr()


def _host_tensor(ptr: int, nbytes: int) -> torch.Tensor:
    arr = np.ctypeslib.as_array(ctypes.cast(ctypes.c_void_p(ptr), ctypes.POINTER(ctypes.c_uint8)), shape=(nbytes,))
    return torch.from_numpy(arr)


class PinnedPool:
    """Pre-allocated pool of equal host slabs; never grows."""

    def __init__(self, total_mb: int = 8192, slab_mb: int = 256, alignment: int = 512, pinned: bool | None = None) -> None:
        if total_mb <= 0:
            raise ValueError(f"total_mb must be positive, got {total_mb}")
        if slab_mb <= 0:
            raise ValueError(f"slab_mb must be positive, got {slab_mb}")
        if total_mb % slab_mb != 0:
            raise ValueError(f"total_mb ({total_mb}) must be evenly divisible by slab_mb ({slab_mb})")
        raw = slab_mb * 1024 * 1024
        self._slab_bytes = (raw + alignment - 1) // alignment * alignment if alignment > 0 else raw
        self._slab_mb = slab_mb
        self._alignment = alignment
        self._num_slabs = total_mb // slab_mb
        self._pool_id = id(self)
        use_pin = torch.cuda.is_available() if pinned is None else bool(pinned)
        handle = ctypes.c_void_p()
        _native.call("sh_pool_create", self._num_slabs, self._slab_bytes, int(use_pin), ctypes.byref(handle))
        self._handle = handle
        self._pinned = use_pin
        _native.track(self, _native.CLOSE_POOL, "shutdown")
        self._slabs: list[PinnedSlab] = []
        for i in range(self._num_slabs):
            ptr = ctypes.c_void_p()
            _native.call("sh_pool_slab_ptr", handle, i, ctypes.byref(ptr))
            self._slabs.append(PinnedSlab(i, _host_tensor(ptr.value, self._slab_bytes), self._slab_bytes, self._pool_id))
        log.info("PinnedPool: %d slabs x %d MiB = %d MiB (pinned=%s)", self._num_slabs, slab_mb, total_mb, use_pin)

    # ── acquire / release ────────────────────────────────────────────

    def _acquire_one(self) -> PinnedSlab:
        if self._handle is None:
            raise RuntimeError("PinnedPool has been shut down")
        slab = ctypes.c_uint32()
        waited = ctypes.c_double()
        _native.call("sh_pool_acquire", self._handle, -1, ctypes.byref(slab), ctypes.byref(waited))
        if waited.value >= _WARN_MS:
            log.warning("PinnedPool.acquire: waited %.1f ms for a free slab", waited.value)
        return self._slabs[slab.value]

    def acquire(self, size_bytes: int) -> PinnedSlab | list[PinnedSlab]:
        needed = max(1, math.ceil(size_bytes / self._slab_bytes))
        if needed > self._num_slabs:
            raise StagehandOOMError(
                f"Requested {size_bytes} bytes ({needed} slabs) exceeds pool capacity of {self._num_slabs} slabs "
                f"({self._num_slabs * self._slab_bytes} bytes)"
            )
        got = [self._acquire_one() for _ in range(needed)]
        return got[0] if needed == 1 else got

    def _check(self, s: PinnedSlab) -> None:
        if s.pool_id != self._pool_id:
            raise AssertionError(f"Slab pool_id {s.pool_id} does not match pool {self._pool_id}")

    def release(self, slab: PinnedSlab | list[PinnedSlab]) -> None:
        for s in ([slab] if isinstance(slab, PinnedSlab) else list(slab)):
            self._check(s)
            if self._handle is not None:
                _native.call("sh_pool_release", self._handle, s.slab_id)

    def release_after(self, slab: PinnedSlab | list[PinnedSlab], stream_handle: int) -> None:
        """Return slab(s) once the work queued so far on ``stream_handle`` completes."""
        for s in ([slab] if isinstance(slab, PinnedSlab) else list(slab)):
            self._check(s)
            if self._handle is not None:
                _native.call("sh_pool_release_after", self._handle, s.slab_id, stream_handle)

    # ── stats / lifecycle ────────────────────────────────────────────

    def native_stats(self) -> dict[str, float]:
        st = np.zeros(1, dtype=POOL_STATS_DTYPE)
        if self._handle is None:
            return {k: 0 for k in POOL_STATS_DTYPE.names}
        _native.call("sh_pool_get_stats", self._handle, st.ctypes.data)
        return {k: st[0][k].item() for k in POOL_STATS_DTYPE.names}

    def stats(self) -> dict[str, int | float]:
        s = self.native_stats()
        return {
            "total": int(s["total"]) if self._handle is not None else 0,
            "free": int(s["free"]),
            "in_use": int(s["in_use"]),
            "peak_in_use": int(s["peak_in_use"]),
            "wait_count": int(s["wait_count"]),
            "total_wait_ms": float(s["total_wait_ms"]),
        }

    def shutdown(self) -> None:
        if getattr(self, "_handle", None) is None:
            return
        for s in self._slabs:
            s.buffer = None  # type: ignore[assignment]
        self._slabs = []
        handle, self._handle = self._handle, None
        _native.call("sh_pool_destroy", handle)

    def __del__(self) -> None:
        try:
            self.shutdown()
        except Exception:
            pass

    @property
    def slab_bytes(self) -> int:
        return self._slab_bytes

    @property
    def num_slabs(self) -> int:
        return self._num_slabs

    @property
    def pinned(self) -> bool:
        return self._pinned

    @property
    def handle(self) -> ctypes.c_void_p | None:
        return self._handle
