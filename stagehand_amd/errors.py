"""Exception hierarchy of the streaming runtime.

Same classes and meanings as the reference (src/stagehand/errors.py:13-30).
``TransferError`` is raised here when a native copy fails, which the
reference declares but never raises.
"""
from __future__ import annotations

__all__ = [
    "StagehandError",
    "StagehandOOMError",
    "DtypeMismatchError",
    "InvalidStateTransitionError",
    "TransferError",
]


class StagehandError(Exception):
    """Base exception for all stagehand errors."""


class StagehandOOMError(StagehandError):
    """Block too large for the pinned pool."""


class DtypeMismatchError(StagehandError):
    """Strict bf16 enforcement violation."""


class InvalidStateTransitionError(StagehandError):
    """Illegal residency state machine transition."""


class TransferError(StagehandError):
    """Async H2D/D2H copy failure."""
