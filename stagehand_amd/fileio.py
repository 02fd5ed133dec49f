"""Weight-file reader over the native ``sh_file_*`` entry points.

The reference reads file-backed parameters through an ``mmap``: one
``torch.frombuffer`` view per tensor, copied into the pinned slab
(src/stagehand/scheduler.py:184-241, 564-601). With
``StagehandConfig.file_reader`` set to ``"pread"`` or ``"direct"``, a block's
tensors become :class:`FileRange` pieces instead, which the native loader reads
straight into its pinned slabs on the host copy threads:

* ``"pread"`` — buffered ``pread`` in pieces of at most 8 MiB; the page cache
  still holds the file, so later steps read it from memory;
* ``"direct"`` — the file is also opened with ``O_DIRECT`` and read around the
  page cache (for models larger than host memory, or read once): into the
  destination by the storage DMA where the kernel can pin it, else through a
  per-thread bounce buffer (pinned slabs from ``hipHostMalloc`` take this
  route: the GPU driver maps them and the kernel refuses to pin them again).

The loader also asks the kernel to read ahead the buffered ranges of the next
queued block.
"""
from __future__ import annotations

import ctypes
import os
import threading
from dataclasses import dataclass

import numpy as np
import torch

from stagehand_amd import _native

__all__ = ["WeightFile", "FileRange", "FileCache", "ALIGN"]

ALIGN = _native.SH_FILE_ALIGN


class WeightFile:
    """An open weight file (a native ``sh_file``)."""

    def __init__(self, path: str | os.PathLike, direct: bool = False) -> None:
        self.path = str(path)
        h = ctypes.c_void_p()
        flags = _native.SH_FILE_DIRECT if direct else 0
        _native.call("sh_file_open", self.path.encode(), flags, ctypes.byref(h))
        self._h: int | None = h.value
        _native.track(self, _native.CLOSE_LEAF)
        self.size = self.info()["size"]

    @property
    def handle(self) -> int:
        if self._h is None:
            raise RuntimeError(f"weight file {self.path} is closed")
        return self._h

    def info(self) -> dict[str, int]:
        out = np.zeros(1, dtype=_native.FILE_INFO_DTYPE)
        _native.call("sh_file_get_info", self.handle, out.ctypes.data)
        return {k: int(out[0][k]) for k in _native.FILE_INFO_DTYPE.names}

    @property
    def direct(self) -> bool:
        return bool(self.info()["direct"])

    def advise_willneed(self, offset: int = 0, nbytes: int = 0) -> None:
        _native.call("sh_file_advise", self.handle, offset, nbytes, _native.SH_FILE_WILLNEED)

    def advise_dontneed(self, offset: int = 0, nbytes: int = 0) -> None:
        """Drops the file's clean pages from the page cache (a cold start for the next read)."""
        _native.call("sh_file_advise", self.handle, offset, nbytes, _native.SH_FILE_DONTNEED)

    def read_into(self, dst: torch.Tensor, offset: int, nbytes: int | None = None, threads: int = 8) -> torch.Tensor:
        """Reads ``nbytes`` (default: all of ``dst``) at ``offset`` into the contiguous host tensor ``dst``."""
        if dst.device.type != "cpu" or not dst.is_contiguous():
            raise ValueError("read_into needs a contiguous host tensor")
        n = dst.numel() * dst.element_size() if nbytes is None else int(nbytes)
        if n > dst.numel() * dst.element_size():
            raise ValueError(f"{n} bytes do not fit a destination of {dst.numel() * dst.element_size()} bytes")
        r = np.zeros(1, dtype=_native.FILE_RANGE_DTYPE)
        r[0] = (self.handle, offset, n, 0)
        _native.call("sh_file_read_batch", r.ctypes.data, 1, dst.data_ptr(), threads)
        return dst

    def close(self) -> None:
        if self._h is not None:
            _native.call("sh_file_close", self._h)
            self._h = None

    def __del__(self) -> None:  # pragma: no cover - interpreter shutdown order
        try:
            self.close()
        except Exception:
            pass


@dataclass(frozen=True)
class FileRange:
    """``nbytes`` at ``offset`` of ``file``: a block-source piece read by the loader."""

    file: WeightFile
    offset: int
    nbytes: int

    def numel(self) -> int:  # byte count, like a uint8 tensor piece
        return self.nbytes


class FileCache:
    """Open weight files by path, one per (path, direct) pair, closed together."""

    def __init__(self) -> None:
        self._files: dict[tuple[str, bool], WeightFile] = {}
        self._lock = threading.Lock()

    def get(self, path: str, direct: bool) -> WeightFile:
        key = (str(path), bool(direct))
        with self._lock:
            f = self._files.get(key)
            if f is None:
                f = WeightFile(key[0], direct=key[1])
                self._files[key] = f
            return f

    def files(self) -> list[WeightFile]:
        with self._lock:
            return list(self._files.values())

    def close(self) -> None:
        with self._lock:
            files, self._files = list(self._files.values()), {}
        for f in files:
            f.close()
