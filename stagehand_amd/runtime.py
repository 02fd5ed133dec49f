"""Block-mode runtime and the one-line layer-mode API.

``StagehandRuntime`` wires registry → pinned pool → residency → budget →
guards → telemetry → transfer engine → scheduler exactly as
src/stagehand/__init__.py:108-205 does, installs the same forward/backward
hooks (:452-548) and exposes the same conversions (:230-275), step calls
(:209-228) and shutdown (:552-595). ``layer()`` / ``wrap()`` / ``Runtime``
are the reference's layer-mode entry points (:621-675).

The transfer engine here owns a native copy stream at the default priority
and a native block loader; see ``stagehand_amd.transfer``.
"""
from __future__ import annotations

import logging
import os
from contextlib import contextmanager
from typing import Generator

import torch
from torch import nn

from stagehand_amd.budget import BudgetManager
from stagehand_amd.config import StagehandConfig
from stagehand_amd.guards import NumericGuard
from stagehand_amd.layer import LayerRuntime
from stagehand_amd.pool import PinnedPool
from stagehand_amd.registry import BlockRegistry
from stagehand_amd.residency import ResidencyMap
from stagehand_amd.scheduler import StagehandScheduler, StaticLookaheadPolicy
from stagehand_amd.telemetry import StagehandTelemetry
from stagehand_amd.transfer import AsyncTransferEngine

__all__ = ["StagehandRuntime", "layer", "wrap", "Runtime"]

log = logging.getLogger(__name__)
_DEBUG_SHUTDOWN = str(os.getenv("SERENITY_DEBUG_STAGEHAND_SHUTDOWN", "0")).strip().lower() in {"1", "true", "yes", "on"}


def _first_tensor(output: object) -> torch.Tensor | None:
    if isinstance(output, torch.Tensor):
        return output
    if isinstance(output, (tuple, list)) and output and isinstance(output[0], torch.Tensor):
        return output[0]
    return None


class StagehandRuntime:
    def __init__(
        self,
        model: nn.Module,
        config: StagehandConfig,
        block_pattern: str = r".*\.block\.\d+$",
        group: str = "transformer",
        dtype: torch.dtype = torch.bfloat16,
        inference_mode: bool = False,
        pool: PinnedPool | None = None,
    ) -> None:
        self._model = model
        self._config = config
        self._inference_mode = inference_mode
        self._registry = BlockRegistry()
        self._registry.build_from_model(model, block_pattern=block_pattern, group=group, dtype=dtype)
        self._pool = pool if pool is not None else PinnedPool(total_mb=config.pinned_pool_mb, slab_mb=config.pinned_slab_mb,
                                                              alignment=config.pinned_slab_alignment)
        self._registry.validate(pool_capacity_bytes=self._pool.num_slabs * self._pool.slab_bytes)
        self._residency = ResidencyMap(self._registry)
        self._budget = BudgetManager(high_watermark_mb=config.vram_high_watermark_mb,
                                     low_watermark_mb=config.vram_low_watermark_mb)
        self._guards: NumericGuard | None = None
        if config.nan_inf_check or config.strict_bf16:
            self._guards = NumericGuard(strict_bf16=config.strict_bf16, fail_on_dtype_promotion=config.fail_on_dtype_promotion,
                                        nan_inf_check=config.nan_inf_check)
        self._telemetry = StagehandTelemetry(enabled=config.telemetry_enabled, interval_steps=config.telemetry_interval_steps,
                                             output_file=config.telemetry_file if config.telemetry_enabled else None)
        self._engine = AsyncTransferEngine(pool=self._pool, max_inflight=config.max_inflight_transfers,
                                           pin_sources=config.pinned_source_cache)
        self._scheduler = StagehandScheduler(
            registry=self._registry, residency=self._residency, transfer_engine=self._engine, budget=self._budget,
            policy=StaticLookaheadPolicy(prefetch_window=config.prefetch_window_blocks,
                                         eviction_cooldown_steps=config.eviction_cooldown_steps),
            guards=self._guards, telemetry=self._telemetry, config=config, inference_mode=inference_mode,
        )
        self._vmm = None
        self._vmm_active_blocks: dict[str, int] = {}
        self._recomputing: set[str] = set()
        log.info("StagehandRuntime: %d blocks registered, pool=%dMB, inference=%s", len(self._registry),
                 config.pinned_pool_mb, inference_mode)

    # ── step lifecycle ───────────────────────────────────────────────

    def begin_step(self, step: int) -> None:
        self._scheduler.begin_step(step)

    def end_step(self) -> None:
        st = self._pool.stats()
        self._telemetry.record_pool_stats(free=int(st["free"]), in_use=int(st["in_use"]))
        self._telemetry.record_vram(used_mb=self._budget.vram_used_mb(), reserved_mb=self._budget.vram_reserved_mb())
        self._scheduler.end_step()

    def convert_registry_to_file_backed(self, source_path: str) -> int:
        n = self._registry.convert_to_file_backed(source_path)
        self._scheduler.refresh_registry_snapshot()
        log.info("StagehandRuntime: converted %d params to file-backed source (%s)", n, source_path)
        return n

    def convert_registry_to_squareq_v2_backed(self, safetensors_path: str, manifest_path: str) -> int:
        n = self._registry.convert_to_squareq_v2_backed(safetensors_path, manifest_path)
        self._scheduler.refresh_registry_snapshot()
        log.info("StagehandRuntime: converted %d params to SquareQ V2-backed source (%s)", n, safetensors_path)
        return n

    def convert_registry_to_file_backed_sharded(self, source_dir: str) -> int:
        n = self._registry.convert_to_file_backed_sharded(source_dir)
        self._scheduler.refresh_registry_snapshot()
        log.info("StagehandRuntime: converted %d params to sharded file-backed source (%s)", n, source_dir)
        return n

    # ── hooks ────────────────────────────────────────────────────────

    # A forward of a block during the backward phase while its backward pre-hook
    # holds it is an activation-checkpoint recompute: the block is already
    # resident and referenced, and the recompute may stop before the block's
    # forward returns (non-reentrant checkpointing stops once it has rebuilt the
    # tensors it needs), so its forward post-hook may never run. Such forwards
    # take no reference of their own; the backward post-hook ends them.

    def _make_pre_forward_hook(self, block_id: str):
        def hook(module: nn.Module, args: tuple) -> None:
            if self._scheduler.in_backward_phase and self._residency.get_entry(block_id).refcount > 0:
                self._recomputing.add(block_id)
                return
            self._scheduler.before_block(block_id)
        return hook

    def _make_post_forward_hook(self, block_id: str):
        def hook(module: nn.Module, args: tuple, output: object) -> None:
            if block_id in self._recomputing:
                self._recomputing.discard(block_id)
                return
            self._scheduler.after_block(block_id, _first_tensor(output))
        return hook

    def _make_pre_backward_hook(self, block_id: str):
        def hook(module: nn.Module, grad_output: tuple) -> None:
            self._scheduler.enter_backward_phase()
            self._scheduler.before_block(block_id)
        return hook

    def _make_post_backward_hook(self, block_id: str):
        def hook(module: nn.Module, grad_input: tuple, grad_output: tuple) -> None:
            self._recomputing.discard(block_id)
            self._scheduler.after_block(block_id)
        return hook

    @contextmanager
    def managed_forward(self) -> Generator[None, None, None]:
        handles = []
        for entry in self._registry.blocks_in_order():
            module = entry.module_ref()
            if module is None:
                continue
            handles.append(module.register_forward_pre_hook(self._make_pre_forward_hook(entry.block_id)))
            handles.append(module.register_forward_hook(self._make_post_forward_hook(entry.block_id)))
        try:
            yield
        finally:
            self._scheduler.exit_backward_phase()
            self._recomputing.clear()
            for h in handles:
                h.remove()

    def set_defer_backward_eviction(self, enabled: bool) -> None:
        self._scheduler.set_defer_backward_eviction(enabled)

    @contextmanager
    def managed_backward(self) -> Generator[None, None, None]:
        if self._inference_mode:
            yield
            return
        handles = []
        for entry in reversed(self._registry.blocks_in_order()):
            module = entry.module_ref()
            if module is None:
                continue
            handles.append(module.register_full_backward_pre_hook(self._make_pre_backward_hook(entry.block_id)))
            handles.append(module.register_full_backward_hook(self._make_post_backward_hook(entry.block_id)))
        try:
            yield
        finally:
            for h in handles:
                h.remove()

    # ── shutdown ─────────────────────────────────────────────────────

    def shutdown(self) -> None:
        if _DEBUG_SHUTDOWN:
            print("[stagehand/debug] runtime.shutdown: engine drain start", flush=True)
        self._engine.shutdown()
        self._scheduler.close()
        self._pool.shutdown()
        self._telemetry.close()

    def shutdown_keep_pool(self) -> PinnedPool:
        self._engine.shutdown()
        self._scheduler.close()
        self._telemetry.close()
        return self._pool

    # ── properties ───────────────────────────────────────────────────

    @property
    def telemetry(self) -> StagehandTelemetry:
        return self._telemetry

    @property
    def stats(self) -> dict:
        return {"pool": self._pool.stats(),
                "telemetry": {"hit_rate": self._telemetry.hit_rate(), "mean_stall_ms": self._telemetry.mean_stall_ms()}}

    @property
    def registry(self) -> BlockRegistry:
        return self._registry

    @property
    def residency(self) -> ResidencyMap:
        return self._residency

    @property
    def scheduler(self) -> StagehandScheduler:
        return self._scheduler

    @property
    def engine(self) -> AsyncTransferEngine:
        return self._engine


def layer(model: nn.Module, *, vram_budget: str | int | None = None, ram_budget: str | int | None = None,
          prefetch_k: int = 3, dtype: torch.dtype = torch.bfloat16, inference_mode: bool = False, telemetry: bool = True,
          pool: PinnedPool | None = None) -> nn.Module:
    """Layer mode on any model: returns the model with hooks and ``_stagehand_layer_runtime`` set."""
    runtime = LayerRuntime(model, vram_budget=vram_budget, ram_budget=ram_budget, prefetch_k=prefetch_k, dtype=dtype,
                           inference_mode=inference_mode, telemetry=telemetry, pool=pool)
    model._stagehand_layer_runtime = runtime  # type: ignore[attr-defined]
    return model


def wrap(model: nn.Module, **kwargs: object) -> nn.Module:
    return layer(model, **kwargs)  # type: ignore[arg-type]


class Runtime:
    """Holds layer-mode keyword arguments: ``Runtime(vram_budget="4GB").layer(model)``."""

    def __init__(self, **kwargs: object) -> None:
        self._kwargs = kwargs

    def layer(self, model: nn.Module) -> nn.Module:
        return layer(model, **self._kwargs)  # type: ignore[arg-type]

    def wrap(self, model: nn.Module) -> nn.Module:
        return wrap(model, **self._kwargs)
