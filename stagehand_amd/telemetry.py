"""Per-step counters of the streaming path (fields of src/stagehand/telemetry.py:24-43).

The scheduler increments the same counters at the same points as the
reference (h2d/d2h bytes, stalls, evictions, prefetch hits/misses). The
reference declares ``copy_time_ms`` but never fills it in; here
``record_copy_time`` fills it with the device time of the step's H2D copies
and unpack kernels when the runtime is asked to time them.
"""
from __future__ import annotations

import json
import logging
from collections import deque
from dataclasses import asdict, dataclass
from typing import IO

__all__ = ["StepMetrics", "StagehandTelemetry"]

log = logging.getLogger(__name__)


@dataclass
class StepMetrics:
    step: int = 0
    h2d_bytes: int = 0
    d2h_bytes: int = 0
    copy_time_ms: float = 0.0
    compute_time_ms: float = 0.0
    stall_time_ms: float = 0.0
    stall_count: int = 0
    evictions: int = 0
    prefetch_hits: int = 0
    prefetch_misses: int = 0
    vram_used_mb: float = 0.0
    vram_reserved_mb: float = 0.0
    host_pool_free: int = 0
    host_pool_in_use: int = 0
    dtype_promotions: int = 0
    nan_count: int = 0
    inf_count: int = 0


class StagehandTelemetry:
    """Collects StepMetrics, keeps a 100-step window, optionally appends JSONL."""

    def __init__(self, enabled: bool = True, interval_steps: int = 10, output_file: str | None = None) -> None:
        self._enabled = enabled
        self._interval_steps = interval_steps
        self._history: deque[StepMetrics] = deque(maxlen=100)
        self._current: StepMetrics | None = None
        self._file_handle: IO[str] | None = open(output_file, "a") if (output_file and enabled) else None  # noqa: SIM115

    def begin_step(self, step: int) -> None:
        if self._enabled:
            self._current = StepMetrics(step=step)

    def end_step(self) -> None:
        if not self._enabled or self._current is None:
            return
        m = self._current
        self._history.append(m)
        if self._file_handle is not None:
            self._file_handle.write(json.dumps(asdict(m)) + "\n")
            self._file_handle.flush()
        if self._interval_steps > 0 and m.step % self._interval_steps == 0:
            log.info(self._format_log_line(m))
        self._current = None

    @property
    def current(self) -> StepMetrics | None:
        return self._current

    @property
    def history(self) -> list[StepMetrics]:
        return list(self._history)

    def record_h2d(self, size_bytes: int) -> None:
        if self._current is not None:
            self._current.h2d_bytes += size_bytes

    def record_d2h(self, size_bytes: int) -> None:
        if self._current is not None:
            self._current.d2h_bytes += size_bytes

    def record_stall(self, duration_ms: float) -> None:
        if self._current is not None:
            self._current.stall_time_ms += duration_ms
            self._current.stall_count += 1

    def record_eviction(self) -> None:
        if self._current is not None:
            self._current.evictions += 1

    def record_prefetch_hit(self) -> None:
        if self._current is not None:
            self._current.prefetch_hits += 1

    def record_prefetch_miss(self) -> None:
        if self._current is not None:
            self._current.prefetch_misses += 1

    def record_nan_inf(self, nan_count: int, inf_count: int) -> None:
        if self._current is not None:
            self._current.nan_count += nan_count
            self._current.inf_count += inf_count

    def record_vram(self, used_mb: float, reserved_mb: float) -> None:
        if self._current is not None:
            self._current.vram_used_mb = used_mb
            self._current.vram_reserved_mb = reserved_mb

    def record_pool_stats(self, free: int, in_use: int) -> None:
        if self._current is not None:
            self._current.host_pool_free = free
            self._current.host_pool_in_use = in_use

    def record_copy_time(self, ms: float) -> None:
        if self._current is not None:
            self._current.copy_time_ms += ms

    def hit_rate(self) -> float:
        hits = sum(m.prefetch_hits for m in self._history)
        total = hits + sum(m.prefetch_misses for m in self._history)
        return hits / total if total else 0.0

    def mean_stall_ms(self) -> float:
        return sum(m.stall_time_ms for m in self._history) / len(self._history) if self._history else 0.0

    def max_stall_ms(self) -> float:
        return max((m.stall_time_ms for m in self._history), default=0.0)

    def vram_trend(self) -> str:
        if len(self._history) < 3:
            return "stable"
        h = list(self._history)
        mid = len(h) // 2
        first = sum(m.vram_used_mb for m in h[:mid]) / mid
        second = sum(m.vram_used_mb for m in h[mid:]) / (len(h) - mid)
        delta = second - first
        return "growing" if delta > 50.0 else "shrinking" if delta < -50.0 else "stable"

    def _format_log_line(self, m: StepMetrics) -> str:
        return (f"[STAGEHAND step={m.step}] hit={self.hit_rate() * 100.0:.1f}% stall={m.stall_time_ms:.1f}ms "
                f"evict={m.evictions} vram={m.vram_used_mb / 1024.0:.1f}G "
                f"pool={m.host_pool_free}/{m.host_pool_free + m.host_pool_in_use}")

    def close(self) -> None:
        if self._file_handle is not None:
            self._file_handle.flush()
            self._file_handle.close()
            self._file_handle = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass
