"""VRAM watermark predicates over torch's allocator statistics
(semantics of src/stagehand/budget.py:18-97).

Block buffers are torch tensors, so ``torch.cuda.memory_allocated`` sees every
byte the streaming path holds on the device, including device staging buffers
of in-flight SquareQ loads. The value is read from the allocator's nested
statistics (``memory_stats_as_nested_dict``), the same counter without the
flattening of every statistic that ``memory_allocated`` does on each call
(about 0.1 ms, and the scheduler asks several times per block). Code that
replaces ``torch.cuda.memory_allocated`` (the reference's tests patch it) is
still what the budget reads.
"""
from __future__ import annotations

from typing import Callable

import torch

__all__ = ["BudgetManager"]

_TORCH_MEMORY_ALLOCATED = torch.cuda.memory_allocated


def _allocated_bytes() -> int:
    fn = torch.cuda.memory_allocated
    if fn is not _TORCH_MEMORY_ALLOCATED:
        return int(fn())
    stats = torch.cuda.memory_stats_as_nested_dict()
    return int(stats.get("allocated_bytes", {}).get("all", {}).get("current", 0))


class BudgetManager:
    def __init__(self, high_watermark_mb: int = 22000, low_watermark_mb: int = 18000) -> None:
        if high_watermark_mb <= low_watermark_mb:
            raise ValueError(
                f"high_watermark_mb ({high_watermark_mb}) must be greater than low_watermark_mb ({low_watermark_mb})"
            )
        self._high_watermark_mb = high_watermark_mb
        self._low_watermark_mb = low_watermark_mb
        self._releasing: Callable[[], int] | None = None

    def count_as_released(self, releasing_bytes: Callable[[], int] | None) -> None:
        """Bytes ``releasing_bytes()`` returns are left out of the used figure: device memory
        that evicted blocks gave up but that asynchronous save-back copies still hold until
        they complete. The reference's synchronous save-back frees it before the next check."""
        self._releasing = releasing_bytes

    def vram_used_mb(self) -> float:
        if not torch.cuda.is_available():
            return 0.0
        used = _allocated_bytes()
        if self._releasing is not None:
            used = max(0, used - int(self._releasing()))
        return used / (1024 * 1024)

    def vram_reserved_mb(self) -> float:
        if not torch.cuda.is_available():
            return 0.0
        return torch.cuda.memory_reserved() / (1024 * 1024)

    def above_high_watermark(self) -> bool:
        return self.vram_used_mb() >= self._high_watermark_mb

    def below_low_watermark(self) -> bool:
        return self.vram_used_mb() < self._low_watermark_mb

    def headroom_mb(self) -> float:
        return self._high_watermark_mb - self.vram_used_mb()

    def should_evict(self) -> bool:
        return self.above_high_watermark()

    def can_prefetch(self) -> bool:
        return not self.above_high_watermark()

    @property
    def high_watermark_mb(self) -> int:
        return self._high_watermark_mb

    @property
    def low_watermark_mb(self) -> int:
        return self._low_watermark_mb

    def __repr__(self) -> str:
        return (f"BudgetManager(high={self._high_watermark_mb}MB, low={self._low_watermark_mb}MB, "
                f"used={self.vram_used_mb():.0f}MB)")
