"""Device-side slab unpack: SquareQ INT8→bf16 dequant and fp32→bf16 cast.

Python face of the ``sh_plan_*`` / ``sh_unpack`` entry points. A plan is a
descriptor table (one row per parameter region, see
``include/stagehand_native.h``) uploaded once; each launch then scatters a
device-resident packed source slab into a contiguous destination buffer laid
out like the reference's block buffers (src/stagehand/scheduler.py:148-165).

Torch owns every device buffer; this module passes raw pointers and sizes and
launches on the caller's current torch stream unless another stream is given.
There is no CPU path: without the native library or a GPU these functions raise.
"""
from __future__ import annotations

import ctypes
from typing import Iterable, Sequence

import numpy as np
import torch

from stagehand_amd import _native
from stagehand_amd._native import (
    DESC_DTYPE,
    KIND_BF16_F32,
    KIND_COPY_BYTES,
    KIND_F32_BF16,
    KIND_I8_ROWSCALE_BF16,
    KIND_I8_ROWSCALE_F32,
    KIND_ZERO_BYTES,
    PLAN_INFO_DTYPE,
)

__all__ = [
    "UnpackPlan",
    "make_descs",
    "dequant_i8_rowscale_bf16",
    "unpack_cast_f32_bf16",
    "unpack_noalloc",
    "KIND_I8_ROWSCALE_BF16",
    "KIND_I8_ROWSCALE_F32",
    "KIND_F32_BF16",
    "KIND_BF16_F32",
    "KIND_COPY_BYTES",
    "KIND_ZERO_BYTES",
]


def make_descs(rows: Iterable[Sequence[int]]) -> np.ndarray:
    """Build a descriptor table from ``(kind, src_off, dst_off, rows, cols, src_ld, scale_off)`` tuples."""
    items = list(rows)
    table = np.zeros(len(items), dtype=DESC_DTYPE)
    for i, (kind, src_off, dst_off, nrows, ncols, src_ld, scale_off) in enumerate(items):
        table[i]["kind"] = kind
        table[i]["src_off"] = src_off
        table[i]["dst_off"] = dst_off
        table[i]["rows"] = nrows
        table[i]["cols"] = ncols
        table[i]["src_ld"] = src_ld
        table[i]["scale_off"] = scale_off
    return table


def _device_ptr(t: torch.Tensor | None, what: str) -> tuple[int, int]:
    if t is None:
        return 0, 0
    if t.device.type != "cuda":
        raise ValueError(f"{what} must be a device tensor, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous")
    return t.data_ptr(), t.numel() * t.element_size()


def _stream_handle(stream: torch.cuda.Stream | int | None) -> int:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


class UnpackPlan:
    """A descriptor table resident on the current device."""

    def __init__(self, descs: np.ndarray) -> None:
        table = np.ascontiguousarray(descs, dtype=DESC_DTYPE)
        self._lib = _native.lib()
        if torch.cuda.is_available():
            _native.call("sh_set_device", torch.cuda.current_device())
        handle = ctypes.c_void_p()
        _native.call("sh_plan_create", table.ctypes.data, len(table), ctypes.byref(handle))
        self._handle = handle
        _native.track(self, _native.CLOSE_LEAF)
        info = np.zeros(1, dtype=PLAN_INFO_DTYPE)
        _native.call("sh_plan_get_info", handle, info.ctypes.data)
        self.info = {name: int(info[0][name]) for name in PLAN_INFO_DTYPE.names}

    @property
    def handle(self) -> ctypes.c_void_p:
        if self._handle is None:
            raise RuntimeError("UnpackPlan has been closed")
        return self._handle

    def close(self) -> None:
        if getattr(self, "_handle", None) is not None:
            _native.call("sh_plan_destroy", self._handle)
            self._handle = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass

    def run(
        self,
        src: torch.Tensor | None,
        dst: torch.Tensor,
        scales: torch.Tensor | None = None,
        zero_points: torch.Tensor | None = None,
        stream: torch.cuda.Stream | int | None = None,
        entry: str = "sh_unpack",
    ) -> None:
        """Launch the plan: ``dst`` ← unpack(``src``) on ``stream``."""
        sp, sb = _device_ptr(src, "src")
        dp, db = _device_ptr(dst, "dst")
        if scales is not None and scales.dtype != torch.float32:
            raise ValueError("scales must be float32")
        if zero_points is not None and zero_points.dtype != torch.float32:
            raise ValueError("zero_points must be float32")
        cp, cb = _device_ptr(scales, "scales")
        zp, zb = _device_ptr(zero_points, "zero_points")
        n_scale = cb // 4
        if zero_points is not None and zb // 4 < n_scale:
            raise ValueError("zero_points must hold as many entries as scales")
        st = _stream_handle(stream)
        if entry == "sh_unpack":
            _native.call(entry, self.handle, sp, sb, cp or None, zp or None, n_scale, dp, db, st)
        elif entry == "sh_dequant_i8_rowscale_bf16":
            _native.call(entry, self.handle, sp, sb, cp or None, zp or None, n_scale, dp, db, st)
        elif entry == "sh_unpack_cast_f32_bf16":
            _native.call(entry, self.handle, sp, sb, dp, db, st)
        else:
            raise ValueError(f"unknown entry point {entry!r}")


def dequant_i8_rowscale_bf16(
    plan: UnpackPlan,
    src: torch.Tensor,
    scales: torch.Tensor,
    dst: torch.Tensor,
    zero_points: torch.Tensor | None = None,
    stream: torch.cuda.Stream | int | None = None,
) -> None:
    """SquareQ dequant of every region of ``plan`` (all SH_KIND_I8_ROWSCALE_BF16)."""
    plan.run(src, dst, scales, zero_points, stream, entry="sh_dequant_i8_rowscale_bf16")


def unpack_cast_f32_bf16(
    plan: UnpackPlan,
    src: torch.Tensor,
    dst: torch.Tensor,
    stream: torch.cuda.Stream | int | None = None,
) -> None:
    """fp32→bf16 unpack of every region of ``plan`` (all SH_KIND_F32_BF16)."""
    plan.run(src, dst, None, None, stream, entry="sh_unpack_cast_f32_bf16")


def unpack_noalloc(
    descs: np.ndarray,
    src: torch.Tensor | None,
    dst: torch.Tensor,
    scales: torch.Tensor | None = None,
    zero_points: torch.Tensor | None = None,
    stream: torch.cuda.Stream | int | None = None,
) -> None:
    """``dst`` ← unpack(``src``) for the descriptor table ``descs``, allocating no device memory
    (``sh_unpack_noalloc``: the launch table lives in the library's static per-GPU scratch).

    The results equal an :class:`UnpackPlan` of the same table run with ``sh_unpack``. Calls on one
    GPU share the scratch; each call's kernels wait on the device for the previous call's, from
    any stream or thread. A call recorded into a graph is not ordered that way: replays of such a
    graph must not overlap other calls on that GPU."""
    table = np.ascontiguousarray(descs, dtype=DESC_DTYPE)
    sp, sb = _device_ptr(src, "src")
    dp, db = _device_ptr(dst, "dst")
    if scales is not None and scales.dtype != torch.float32:
        raise ValueError("scales must be float32")
    if zero_points is not None and zero_points.dtype != torch.float32:
        raise ValueError("zero_points must be float32")
    cp, cb = _device_ptr(scales, "scales")
    zp, zb = _device_ptr(zero_points, "zero_points")
    n_scale = cb // 4
    if zero_points is not None and zb // 4 < n_scale:
        raise ValueError("zero_points must hold as many entries as scales")
    _native.call("sh_unpack_noalloc", table.ctypes.data if len(table) else None, len(table), sp or None, sb,
                 cp or None, zp or None, n_scale, dp, db, _stream_handle(stream))
