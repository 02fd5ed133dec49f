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
from pathlib import Path
from typing import Generator

import torch
from torch import nn

from stagehand_amd import _native
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


def _hint_hw_queues() -> None:
    """Logs once when HIP runs with fewer than 8 hardware queues (GPU_MAX_HW_QUEUES, 4 by default).
    HIP maps every stream onto those queues, and streams that share one run in the order their
    work was queued: the save-backs' chunk comparisons, on the block loader's unpack stream, then
    run behind compute queued after them, and training steps wait longer on save-backs."""
    global _HW_QUEUES_HINTED
    if _HW_QUEUES_HINTED:
        return
    _HW_QUEUES_HINTED = True
    try:
        queues = int(os.environ.get("GPU_MAX_HW_QUEUES", "4"))
    except ValueError:
        return
    if queues < 8:
        log.info("StagehandRuntime: HIP has %d hardware queues (GPU_MAX_HW_QUEUES); training with changed-chunk "
                 "save-backs runs faster with 8, set before HIP starts", queues)


_HW_QUEUES_HINTED = False


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
                                           pin_sources=config.pinned_source_cache,
                                           save_back=config.save_back_engine)
        if not inference_mode and config.save_back_changed_chunks and torch.cuda.is_available():
            _hint_hw_queues()
        self._scheduler = StagehandScheduler(
            registry=self._registry, residency=self._residency, transfer_engine=self._engine, budget=self._budget,
            policy=StaticLookaheadPolicy(prefetch_window=config.prefetch_window_blocks,
                                         eviction_cooldown_steps=config.eviction_cooldown_steps),
            guards=self._guards, telemetry=self._telemetry, config=config, inference_mode=inference_mode,
        )
        # VMM backend (inference only, as src/stagehand/__init__.py:185-198): blocks
        # registered with vmm_register_model are served from mapped device memory
        self._vmm = None
        self._vmm_model_id: str | None = None
        self._vmm_active_blocks: dict[str, int] = {}
        self._vmm_block_id_to_idx: dict[str, int] = {}
        self._recomputing: set[str] = set()
        self._vmm_saved: dict[str, list] = {}
        if inference_mode and torch.cuda.is_available():
            from stagehand_amd import vmm as _vmm_mod

            if _vmm_mod.is_available():
                try:
                    self._vmm = _vmm_mod.VmmManager(device=torch.cuda.current_device(), engine=self._engine,
                                                    file_reader=getattr(config, "file_reader", "mmap"))
                    for i, entry in enumerate(self._registry.blocks_in_order()):
                        self._vmm_block_id_to_idx[entry.block_id] = i
                except Exception as e:  # noqa: BLE001 — the block-swap path still works
                    log.warning("VMM init failed, using block-swap: %s", e)
                    self._vmm = None
        self._shut_down = False
        _native.track(self, _native.CLOSE_RUNTIME, "shutdown")
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

    # ── VMM (src/stagehand/__init__.py:278-448) ──────────────────────

    def vmm_register_model(self, model_id: str, dtype_str: str = "bfloat16", safetensors_path: str | None = None):
        """Registers every block with the VMM backend (one region per block). Weights come from
        ``safetensors_path`` — a file, or a directory of shards with its index (fully-qualified
        parameter names) — or, without one, from host copies of the module parameters. Returns
        the VmmModelHandle, or None without the backend."""
        if self._vmm is None:
            return None
        ordered = self._registry.blocks_in_order()
        handle = self._vmm.register_model(model_id, [e.size_bytes for e in ordered], dtype_str)
        for i, entry in enumerate(ordered):
            layout = self._block_layout(entry)
            total = sum(numel for *_r, numel in layout)
            if total > 0:
                handle.register_block_shape(i, [total])
        source_ok = False
        if safetensors_path is not None and (str(safetensors_path).endswith(".safetensors")
                                             or Path(safetensors_path).is_dir()):
            names_by_module = {id(m): n for n, m in self._model.named_modules()}
            block_map = []
            for entry in ordered:
                module = entry.module_ref()
                prefix = names_by_module.get(id(module), "") if module is not None else ""
                prefix = prefix + "." if prefix else ""
                block_map.append([prefix + name for name, *_r in self._block_layout(entry)])
            try:
                handle.set_mmap_source(str(safetensors_path), block_map)
                source_ok = True
            except Exception as e:  # noqa: BLE001
                log.warning("VMM: file source failed for %s: %s, falling back to host copies", model_id, e)
        if not source_ok:
            for i, entry in enumerate(ordered):
                module = entry.module_ref()
                layout = self._block_layout(entry)
                if module is None or not layout:
                    continue
                params = dict(module.named_parameters())
                parts = [params[name].data.to(dtype).reshape(-1).view(torch.uint8) for name, _s, dtype, _o, _n in layout
                         if params[name].numel() > 0]
                if parts:
                    handle.set_ram_weights(i, torch.cat(parts).cpu())
        self._vmm.activate_model(model_id)
        self._vmm_model_id = model_id
        log.info("VMM: registered model %s with %d blocks", model_id, len(ordered))
        return handle

    def _block_layout(self, entry) -> list:
        if entry.param_layout:
            return list(entry.param_layout)
        module = entry.module_ref()
        if module is None:
            return []
        from stagehand_amd.scheduler import _build_param_layout

        return _build_param_layout(module, entry.dtype)

    def _vmm_before_block(self, block_id: str, module: nn.Module) -> bool:
        """Serves the block from its VMM region; False sends it down the block-swap path."""
        if self._vmm is None or self._vmm_model_id not in self._vmm.models:
            return False
        idx = self._vmm_block_id_to_idx.get(block_id)
        if idx is None:
            return False
        handle = self._vmm.models[self._vmm_model_id]
        stream = torch.cuda.current_stream().cuda_stream
        tensor, ok = handle.get_block_tensor(idx, stream)
        # the next block's fill runs while this one computes; further blocks of the prefetch
        # window only while they fit under the ceiling without evicting anything
        handle.prefetch_block(idx + 1, stream)
        for k in range(2, self._config.prefetch_window_blocks + 1):
            if not handle.fits_without_eviction(idx + k):
                break
            handle.prefetch_block(idx + k, stream)
        if not ok:
            return False
        try:
            layout = self._block_layout(self._registry.get(block_id))
            if layout:
                from stagehand_amd.scheduler import _get_param_data, _restore_params_from_tensor

                # what the parameters hold now (host tensors of module-resident parameters,
                # the block-swap copy's views, or empty placeholders) comes back after the block
                self._vmm_saved[block_id] = [(name, _get_param_data(module, name)) for name, *_r in layout]
                _restore_params_from_tensor(module, tensor.view(torch.uint8), layout)
        except Exception as e:  # noqa: BLE001
            log.warning("VMM: param restore failed for %s, falling back: %s", block_id, e)
            handle.release_block(idx)
            return False
        self._vmm_active_blocks[block_id] = idx
        self._scheduler._cursor += 1
        self._telemetry.record_prefetch_hit()
        self._scheduler._prefetch_ahead()
        return True

    def _vmm_after_block(self, block_id: str) -> None:
        idx = self._vmm_active_blocks.pop(block_id, None)
        if idx is None:
            return
        entry = self._registry.get(block_id)
        module = entry.module_ref()
        saved = self._vmm_saved.pop(block_id, None)
        if module is not None and saved:
            # the parameter views hold the region's tensor: give the parameters back what
            # they held before the block (the reference empties them, which loses
            # module-resident parameters such as norms and the block-swap copy's views)
            from stagehand_amd.scheduler import _set_param_data

            for name, data in saved:
                _set_param_data(module, name, data)
        if self._vmm_model_id in self._vmm.models:
            self._vmm.models[self._vmm_model_id].release_block(idx)

    @property
    def vmm(self):
        return self._vmm

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
            if self._vmm is not None and self._vmm_before_block(block_id, module):
                return
            self._scheduler.before_block(block_id)
        return hook

    def _make_post_forward_hook(self, block_id: str):
        def hook(module: nn.Module, args: tuple, output: object) -> None:
            if block_id in self._recomputing:
                self._recomputing.discard(block_id)
                return
            if block_id in self._vmm_active_blocks:
                self._vmm_after_block(block_id)
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
        if self._shut_down:
            return
        self._shut_down = True
        if _DEBUG_SHUTDOWN:
            print("[stagehand/debug] runtime.shutdown: engine drain start", flush=True)
        if self._vmm is not None:
            for bid in list(self._vmm_active_blocks):
                self._vmm_after_block(bid)
            self._vmm.shutdown()
            self._vmm = None
        self._engine.shutdown()
        self._scheduler.close()
        self._pool.shutdown()
        self._telemetry.close()

    def shutdown_keep_pool(self) -> PinnedPool:
        self._shut_down = True
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
