"""MI355X-native weight-streaming data path for Stagehand-style block streaming.

Host-side mirror of the reference's streaming runtime (pool, transfer engine,
registry, residency, scheduler) over a C-ABI native library
(``include/stagehand_native.h``) whose HIP kernels do the SquareQ INT8→bf16
dequant and fp32→bf16 slab unpack on the device.
"""
from __future__ import annotations

from stagehand_amd.errors import (
    DtypeMismatchError,
    InvalidStateTransitionError,
    StagehandError,
    StagehandOOMError,
    TransferError,
)

__all__ = [
    "StagehandError",
    "StagehandOOMError",
    "DtypeMismatchError",
    "InvalidStateTransitionError",
    "TransferError",
]
