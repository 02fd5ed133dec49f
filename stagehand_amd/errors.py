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
    """Root of every error this package raises on purpose."""


class StagehandOOMError(StagehandError):
    """A block (or a request of slabs) does not fit the pinned slab pool."""


class DtypeMismatchError(StagehandError):
    """A block produced a dtype other than bf16 while strict bf16 checking is on."""


class InvalidStateTransitionError(StagehandError):
    """A block was asked to move between residency states the FSM does not connect."""


class TransferError(StagehandError):
    """A host-to-device or device-to-host copy failed in the native engine."""
