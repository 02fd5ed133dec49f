"""Block source assembly for the device path.

The reference converts every parameter on the host while copying it into the
pinned slab (casts at src/stagehand/scheduler.py:181, 224-230, 1066-1071;
SquareQ dequant at :290-300; zero fill at :240, :276-297, :325) and sends the
finished runtime-dtype block over PCIe. Here a block is described instead as
raw source pieces plus an unpack plan:

* same-dtype parameters (bf16 → bf16) are byte copies;
* fp32 parameters become SH_KIND_F32_BF16 regions, cast on the device;
* SquareQ weights travel as int8 rows (with the padded row stride of the slab
  format) plus per-row fp32 scales (and zero points when any is non-zero) and
  become SH_KIND_I8_ROWSCALE_* regions, dequantised on the device — half the
  PCIe bytes of a bf16 block;
* missing parameters become zero-fill regions;
* parameters read from a weight file by the native reader are
  :class:`~stagehand_amd.fileio.FileRange` pieces; in a plan layout they are
  placed in file order and neighbours in the file merge into one read.

When every region is a byte copy or zero fill, the slab image equals the
destination image and no kernel runs (``plan is None``: a single H2D copy).
The branch structure of the SquareQ fallbacks is that of
src/stagehand/scheduler.py:243-325; ``oracle/squareq.py`` restates it on the
CPU and the GPU tests compare the two.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Mapping

import numpy as np
import torch

from stagehand_amd.fileio import FileRange
from stagehand_amd.transfer import BlockSource
from stagehand_amd.unpack import (
    KIND_BF16_F32,
    KIND_COPY_BYTES,
    KIND_F32_BF16,
    KIND_I8_ROWSCALE_BF16,
    KIND_I8_ROWSCALE_F32,
    KIND_ZERO_BYTES,
    UnpackPlan,
    make_descs,
)

__all__ = ["SourceBuilder", "PlanCache", "SUPPORTED_RUNTIME_DTYPES"]

SUPPORTED_RUNTIME_DTYPES = (torch.bfloat16, torch.float32)
_ALIGN = 16


def _align(x: int) -> int:
    return (x + _ALIGN - 1) // _ALIGN * _ALIGN


def _host_contig(t: torch.Tensor) -> torch.Tensor:
    t = t.detach()
    if t.device.type != "cpu":
        t = t.to("cpu")
    return t.contiguous()


_ZERO_HOST = torch.zeros(0, dtype=torch.uint8)


def _zeros(nbytes: int) -> torch.Tensor:
    global _ZERO_HOST
    if _ZERO_HOST.numel() < nbytes:
        _ZERO_HOST = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8)
    return _ZERO_HOST[:nbytes]


@dataclass
class SourceBuilder:
    """Collects the regions of one block and lays out its source slab."""

    runtime_dtype: torch.dtype
    dst_bytes: int
    _regions: list[tuple] = field(default_factory=list)  # (kind, dst_off, host tensor|None, rows, cols, ld, scale rows)
    _scales: list[Any] = field(default_factory=list)  # per dequant region: fp32 tensor or FileRange
    _zps: list[Any] = field(default_factory=list)  # per dequant region: fp32 tensor, FileRange or None
    _mutable: list[bool] = field(default_factory=list)  # per region: bytes may change between loads

    def __post_init__(self) -> None:
        if self.runtime_dtype not in SUPPORTED_RUNTIME_DTYPES:
            raise ValueError(f"device path supports runtime dtypes {SUPPORTED_RUNTIME_DTYPES}, got {self.runtime_dtype}")

    # ── regions ──────────────────────────────────────────────────────

    def add_param(self, dst_off: int, value: torch.Tensor, mutable: bool = False) -> None:
        """``dst ← value.to(runtime_dtype)`` (rounded on the device when narrowing).
        ``mutable`` marks module parameters, whose bytes may change between loads."""
        v = _host_contig(value).reshape(-1)
        rt = self.runtime_dtype
        self._mutable.append(mutable)
        if v.dtype == rt:
            self._regions.append((KIND_COPY_BYTES, dst_off, v.view(torch.uint8), 1, v.numel() * v.element_size(), 0, 0))
            return
        if v.dtype == torch.float16:
            v = v.to(torch.float32)  # exact widening; any rounding happens on the device
        if rt == torch.bfloat16 and v.dtype == torch.float32:
            self._regions.append((KIND_F32_BF16, dst_off, v.view(torch.uint8), 1, v.numel(), 0, 0))
        elif rt == torch.float32 and v.dtype == torch.bfloat16:
            self._regions.append((KIND_BF16_F32, dst_off, v.view(torch.uint8), 1, v.numel(), 0, 0))
        elif rt == torch.float32 and v.dtype == torch.float32:
            self._regions.append((KIND_COPY_BYTES, dst_off, v.view(torch.uint8), 1, v.numel() * 4, 0, 0))
        else:
            self._mutable.pop()
            raise ValueError(f"no device conversion from {v.dtype} to {rt}")

    def add_file_param(self, dst_off: int, frange: FileRange, source_dtype: torch.dtype, numel: int) -> bool:
        """``dst ← file bytes.to(runtime_dtype)`` for a tensor stored contiguously in a weight file.
        Returns False (nothing added) for a source dtype the device cannot convert from raw
        bytes; the caller then reads that tensor through a host view."""
        rt = self.runtime_dtype
        if source_dtype == rt:
            kind, cols = KIND_COPY_BYTES, numel * rt.itemsize
        elif rt == torch.bfloat16 and source_dtype == torch.float32:
            kind, cols = KIND_F32_BF16, numel
        elif rt == torch.float32 and source_dtype == torch.bfloat16:
            kind, cols = KIND_BF16_F32, numel
        else:
            return False
        if frange.nbytes != numel * source_dtype.itemsize:
            raise ValueError(f"file range of {frange.nbytes} bytes does not hold {numel} {source_dtype} values")
        self._regions.append((kind, dst_off, frange, 1, cols, 0, 0))
        self._mutable.append(False)
        return True

    def add_zero(self, dst_off: int, nbytes: int) -> None:
        if nbytes > 0:
            self._regions.append((KIND_ZERO_BYTES, dst_off, None, 1, nbytes, 0, 0))
            self._mutable.append(False)

    def add_dequant(self, dst_off: int, q_rows: torch.Tensor, in_flat: int, scale: torch.Tensor,
                    zero_point: torch.Tensor | None) -> None:
        """SquareQ weight: q_rows is the (out, ld) int8 row block, the first in_flat columns are used."""
        q = _host_contig(q_rows)
        if q.dtype != torch.int8:
            raise ValueError(f"SquareQ qweight must be int8, got {q.dtype}")
        out_dim, ld = int(q.shape[0]), int(q.shape[1])
        if in_flat > ld:
            raise ValueError(f"SquareQ row of {ld} values is shorter than in_features {in_flat}")
        kind = KIND_I8_ROWSCALE_BF16 if self.runtime_dtype == torch.bfloat16 else KIND_I8_ROWSCALE_F32
        s = _host_contig(scale).reshape(-1)[:out_dim].to(torch.float32)
        z = None if zero_point is None else _host_contig(zero_point).reshape(-1)[:out_dim].to(torch.float32)
        self._regions.append((kind, dst_off, q.view(torch.uint8).reshape(-1), out_dim, in_flat, ld, out_dim))
        self._scales.append(s)
        self._zps.append(z)
        self._mutable.append(False)

    def add_dequant_file(self, dst_off: int, q_rows: FileRange, out_dim: int, ld: int, in_flat: int,
                         scale: FileRange | torch.Tensor, zero_point: FileRange | torch.Tensor | None) -> None:
        """SquareQ weight read from a file: ``q_rows`` holds ``out_dim`` int8 rows of ``ld`` values
        (the first ``in_flat`` are used); ``scale`` / ``zero_point`` give ``out_dim`` fp32 values
        each, as file ranges or host tensors; ``zero_point`` None means zeros."""
        if in_flat > ld:
            raise ValueError(f"SquareQ row of {ld} values is shorter than in_features {in_flat}")
        if q_rows.nbytes != out_dim * ld:
            raise ValueError(f"int8 range of {q_rows.nbytes} bytes is not {out_dim} rows of {ld}")
        for what, v in (("scale", scale), ("zero point", zero_point)):
            if isinstance(v, FileRange) and v.nbytes != 4 * out_dim:
                raise ValueError(f"{what} range of {v.nbytes} bytes does not hold {out_dim} fp32 values")
        kind = KIND_I8_ROWSCALE_BF16 if self.runtime_dtype == torch.bfloat16 else KIND_I8_ROWSCALE_F32
        if not isinstance(scale, FileRange):
            scale = _host_contig(scale).reshape(-1)[:out_dim].to(torch.float32)
        if zero_point is not None and not isinstance(zero_point, FileRange):
            zero_point = _host_contig(zero_point).reshape(-1)[:out_dim].to(torch.float32)
        self._regions.append((kind, dst_off, q_rows, out_dim, in_flat, ld, out_dim))
        self._scales.append(scale)
        self._zps.append(zero_point)
        self._mutable.append(False)

    # ── layout ───────────────────────────────────────────────────────

    def finish(self) -> tuple[BlockSource, np.ndarray | None]:
        """Returns the block source and, when a kernel is needed, its descriptor table."""
        if all(r[0] in (KIND_COPY_BYTES, KIND_ZERO_BYTES) for r in self._regions):
            pieces = []
            mutable = set()
            for (kind, dst_off, t, _r, nbytes, _ld, _s), mut in zip(self._regions, self._mutable):
                if mut:
                    mutable.add(len(pieces))
                pieces.append((dst_off, t if kind == KIND_COPY_BYTES else _zeros(nbytes)))
            key = repr([(o, t.numel()) for o, t in pieces]).encode() + b"|direct|" + str(self.dst_bytes).encode()
            return BlockSource(pieces=pieces, src_bytes=self.dst_bytes, key=key, mutable=frozenset(mutable)), None

        pieces: list[tuple[int, Any]] = []
        mutable = set()
        rows: list[tuple] = []
        cursor = 0
        # scale rows follow the dequant regions in the order they were added (the order of _scales)
        first_row, scale_row = [], 0
        for r in self._regions:
            first_row.append(scale_row)
            scale_row += r[6]
        # file ranges go first, in file order, so that neighbours in the file are
        # neighbours in the slab (one read each run); the rest keep their order
        order = sorted(range(len(self._regions)), key=lambda i: (
            0, self._regions[i][2].file.path, self._regions[i][2].offset) if isinstance(self._regions[i][2], FileRange)
            else (1, "", i))
        for i in order:
            (kind, dst_off, t, r, c, ld, srows), mut = self._regions[i], self._mutable[i]
            if kind == KIND_ZERO_BYTES:
                rows.append((kind, 0, dst_off, r, c, 0, 0))
                continue
            if isinstance(t, FileRange):
                prev = pieces[-1] if pieces else None
                if (prev is not None and isinstance(prev[1], FileRange) and prev[1].file is t.file
                        and prev[1].offset + prev[1].nbytes == t.offset):
                    off = cursor  # continues the previous range in the file: one read
                    pieces[-1] = (prev[0], FileRange(t.file, prev[1].offset, prev[1].nbytes + t.nbytes))
                else:
                    off = _align(cursor)
                    pieces.append((off, t))
                cursor = off + t.nbytes
            else:
                off = _align(cursor)
                if mut:
                    mutable.add(len(pieces))
                pieces.append((off, t))
                cursor = off + t.numel()
            rows.append((kind, off, dst_off, r, c, ld, first_row[i]))
        scale_off = zp_off = -1
        if self._scales:
            counts = [s.nbytes // 4 if isinstance(s, FileRange) else s.numel() for s in self._scales]
            scale_off = _align(cursor)
            pieces.extend(_row_pieces(scale_off, self._scales, counts))
            cursor = scale_off + 4 * sum(counts)
            # a zero-point range counts as non-zero (the caller passes None for all-zero ones)
            if any(isinstance(z, FileRange) or (z is not None and bool(torch.any(z != 0))) for z in self._zps):
                zp_off = _align(cursor)
                zps = [z if z is not None else torch.zeros(n, dtype=torch.float32) for z, n in zip(self._zps, counts)]
                pieces.extend(_row_pieces(zp_off, zps, counts))
                cursor = zp_off + 4 * sum(counts)
        descs = make_descs(rows)
        key = descs.tobytes() + f"|{scale_off}|{zp_off}|{cursor}".encode()
        src = BlockSource(pieces=pieces, src_bytes=max(cursor, 1), scale_off=scale_off, zp_off=zp_off,
                          n_scale=scale_row, key=key, mutable=frozenset(mutable))
        return src, descs


def _row_pieces(base: int, values: list[Any], counts: list[int]) -> list[tuple[int, Any]]:
    """Per-row fp32 vectors back to back from ``base``: host tensors merge into one piece per
    run, file ranges stay pieces of their own."""
    out: list[tuple[int, Any]] = []
    run: list[torch.Tensor] = []
    run_off = off = base
    for v, n in zip(values, counts):
        if isinstance(v, FileRange):
            if run:
                out.append((run_off, torch.cat(run).view(torch.uint8)))
                run = []
            out.append((off, v))
            run_off = off + 4 * n
        else:
            if not run:
                run_off = off
            run.append(v)
        off += 4 * n
    if run:
        out.append((run_off, torch.cat(run).view(torch.uint8)))
    return out


class PlanCache:
    """Device-resident unpack plans keyed by block; rebuilt when the table changes."""

    def __init__(self) -> None:
        self._plans: dict[str, tuple[bytes, UnpackPlan]] = {}

    def get(self, block_id: str, descs: np.ndarray) -> UnpackPlan:
        key = descs.tobytes()
        hit = self._plans.get(block_id)
        if hit is not None and hit[0] == key:
            return hit[1]
        plan = UnpackPlan(descs)
        if hit is not None:
            hit[1].close()
        self._plans[block_id] = (key, plan)
        return plan

    def clear(self) -> None:
        for _k, plan in self._plans.values():
            try:
                plan.close()
            except Exception:
                pass
        self._plans.clear()


def squareq_weight_tensors(layer: Mapping[str, Any]) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None:
    q, s, z = layer.get("qweight"), layer.get("scale"), layer.get("zero_point")
    if isinstance(q, torch.Tensor) and isinstance(s, torch.Tensor) and isinstance(z, torch.Tensor):
        return q, s, z
    return None
