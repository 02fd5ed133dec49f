"""MI355X-native weight-streaming data path with Stagehand's Python surface.

The public names are those of the reference package (src/stagehand/__init__.py:44-82):
``StagehandRuntime`` (block mode), ``layer()`` / ``wrap()`` / ``Runtime``
(layer mode), the registry, residency map, pinned pool, transfer engine,
scheduler, budget, guards and telemetry types. Underneath, a C-ABI native
library (``include/stagehand_native.h``) owns pinned slabs, copy streams,
events and a block-loader thread, and its HIP kernels do the SquareQ
INT8→bf16 dequant and fp32→bf16 unpack on the device.
"""
from __future__ import annotations

from stagehand_amd.budget import BudgetManager
from stagehand_amd.config import StagehandConfig
from stagehand_amd.errors import (
    DtypeMismatchError,
    InvalidStateTransitionError,
    StagehandError,
    StagehandOOMError,
    TransferError,
)
from stagehand_amd.guards import NumericGuard
from stagehand_amd.layer import LayerRuntime
from stagehand_amd.pool import PinnedPool, PinnedSlab
from stagehand_amd.registry import BlockEntry, BlockRegistry, FileParamSpec, SquareQParamSpec
from stagehand_amd.residency import BlockState, ResidencyEntry, ResidencyMap
from stagehand_amd.runtime import Runtime, StagehandRuntime, layer, wrap
from stagehand_amd.scheduler import StagehandScheduler, StaticLookaheadPolicy
from stagehand_amd.telemetry import StagehandTelemetry, StepMetrics
from stagehand_amd.transfer import AsyncTransferEngine, TransferHandle

__version__ = "0.1.0"

__all__ = [
    "StagehandConfig",
    "DtypeMismatchError",
    "InvalidStateTransitionError",
    "StagehandError",
    "StagehandOOMError",
    "TransferError",
    "PinnedPool",
    "PinnedSlab",
    "BlockEntry",
    "BlockRegistry",
    "FileParamSpec",
    "SquareQParamSpec",
    "BlockState",
    "ResidencyEntry",
    "ResidencyMap",
    "AsyncTransferEngine",
    "TransferHandle",
    "StaticLookaheadPolicy",
    "StagehandScheduler",
    "BudgetManager",
    "NumericGuard",
    "StagehandTelemetry",
    "StepMetrics",
    "StagehandRuntime",
    "LayerRuntime",
    "layer",
    "wrap",
    "Runtime",
]
