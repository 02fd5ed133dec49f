"""Alias module kept for import compatibility (src/stagehand/pinned_pool.py:6)."""
from stagehand_amd.pool import PinnedPool, PinnedSlab  # noqa: F401

__all__ = ["PinnedPool", "PinnedSlab"]
