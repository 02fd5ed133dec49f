"""Layer mode: stream every ``nn.Linear`` / ``nn.Conv2d`` / ``nn.Embedding``.

Lifecycle and sizing follow src/stagehand/layer.py: discovery of leaf layers
with their own parameters (:49-72), budget strings (:75-91), automatic pool
and watermark configuration (:101-165), a trace step with prefetch 0 that
records the execution order (:392-422), then a registry rebuilt in traced
order with ``prefetch_k`` lookahead (:472-520), and auto-step detection when
the first traced layer fires again (:424-440).

On a GPU each layer load is a native block load (pinned slab, copy stream,
fp32→bf16 rounding on the device); non-managed parameters and buffers move
to the device once, as in the reference (:292-306) — their floating-point
cast is torch's own ``.to(dtype)``, outside the streamed path.
"""
from __future__ import annotations

import logging
import math

import torch
from torch import nn

from stagehand_amd import _native
from stagehand_amd.budget import BudgetManager
from stagehand_amd.config import StagehandConfig
from stagehand_amd.guards import NumericGuard
from stagehand_amd.pool import PinnedPool
from stagehand_amd.registry import BlockRegistry
from stagehand_amd.residency import ResidencyMap
from stagehand_amd.scheduler import StagehandScheduler, StaticLookaheadPolicy
from stagehand_amd.telemetry import StagehandTelemetry
from stagehand_amd.transfer import AsyncTransferEngine

__all__ = ["LayerRuntime", "LAYER_TYPES"]

log = logging.getLogger(__name__)

LAYER_TYPES: tuple[type[nn.Module], ...] = (nn.Linear, nn.Conv2d, nn.Embedding)


def _discover_layers(model: nn.Module, target_types: tuple[type[nn.Module], ...] = LAYER_TYPES) -> list[tuple[str, nn.Module]]:
    seen: set[int] = set()
    out: list[tuple[str, nn.Module]] = []
    for name, module in model.named_modules():
        if not name or not isinstance(module, target_types):
            continue
        if not any(True for _ in module.parameters(recurse=False)):
            continue
        if id(module) in seen:
            continue
        seen.add(id(module))
        out.append((name, module))
    return out


def _parse_budget(value: str | int | None) -> int | None:
    if value is None:
        return None
    if isinstance(value, int):
        return value
    v = value.strip().upper()
    if v.endswith("GB"):
        return int(float(v[:-2]) * 1024 ** 3)
    if v.endswith("MB"):
        return int(float(v[:-2]) * 1024 ** 2)
    if v.endswith("B"):
        return int(v[:-1])
    return int(v)


def _next_power_of_two(n: int) -> int:
    return 1 if n <= 0 else 1 << (n - 1).bit_length()


def _auto_pool_config(layers: list[tuple[str, nn.Module]], dtype: torch.dtype, prefetch_k: int,
                      vram_budget: int | None, ram_budget: int | None) -> StagehandConfig:
    """Slab = next power of two MiB ≥ the largest layer at ``dtype``; prefetch_k + 4 slabs;
    watermarks at 80 % / 60 % of the VRAM budget (or the device's memory)."""
    max_layer = max((sum(p.numel() for p in m.parameters(recurse=False)) * dtype.itemsize for _n, m in layers), default=0)
    slab_mb = max(1, _next_power_of_two(math.ceil(max_layer / (1024 * 1024))))
    total_mb = slab_mb * (prefetch_k + 4)
    if ram_budget is not None:
        ram_mb = ram_budget // (1024 * 1024)
        if total_mb > ram_mb:
            total_mb = max(slab_mb, (ram_mb // slab_mb) * slab_mb)
    if vram_budget is not None:
        vram_mb = vram_budget // (1024 * 1024)
        high, low = int(vram_mb * 0.80), int(vram_mb * 0.60)
    elif torch.cuda.is_available():
        vram_mb = torch.cuda.get_device_properties(0).total_memory // (1024 * 1024)
        high, low = int(vram_mb * 0.80), int(vram_mb * 0.60)
    else:
        high, low = 22000, 18000
    if high <= low:
        high = low + 1
    return StagehandConfig(
        pinned_pool_mb=total_mb, pinned_slab_mb=slab_mb, vram_high_watermark_mb=high, vram_low_watermark_mb=low,
        prefetch_window_blocks=prefetch_k, eviction_cooldown_steps=0, nan_inf_check=False, strict_bf16=False,
        fail_on_dtype_promotion=False, telemetry_enabled=True, telemetry_interval_steps=10,
    )


class LayerRuntime:
    def __init__(
        self,
        model: nn.Module,
        vram_budget: str | int | None = None,
        ram_budget: str | int | None = None,
        prefetch_k: int = 3,
        dtype: torch.dtype = torch.bfloat16,
        inference_mode: bool = False,
        telemetry: bool = True,
        pool: PinnedPool | None = None,
    ) -> None:
        self._model = model
        self._dtype = dtype
        self._prefetch_k = prefetch_k
        self._inference_mode = inference_mode
        layers = _discover_layers(model)
        if not layers:
            # the message starts as the reference's does: callers match on "No eligible layers"
            raise ValueError("No eligible layers in the model: layer mode streams nn.Linear, nn.Conv2d and "
                             "nn.Embedding modules, and it found none with parameters.")
        self._layer_map: dict[str, nn.Module] = dict(layers)
        self._all_layer_names = [n for n, _ in layers]
        self._config = _auto_pool_config(layers, dtype, prefetch_k, _parse_budget(vram_budget), _parse_budget(ram_budget))
        self._config.telemetry_enabled = telemetry
        self._pool = pool if pool is not None else PinnedPool(total_mb=self._config.pinned_pool_mb,
                                                              slab_mb=self._config.pinned_slab_mb)
        self._engine = AsyncTransferEngine(pool=self._pool, max_inflight=self._config.max_inflight_transfers,
                                           save_back=self._config.save_back_engine)
        self._budget = BudgetManager(self._config.vram_high_watermark_mb, self._config.vram_low_watermark_mb)
        self._guards: NumericGuard | None = None
        self._telemetry_inst = StagehandTelemetry(enabled=self._config.telemetry_enabled,
                                                  interval_steps=self._config.telemetry_interval_steps, output_file=None)
        self._registry = BlockRegistry()
        self._registry.build_from_module_list(layers, "layer", dtype)
        self._registry.validate(pool_capacity_bytes=self._pool.num_slabs * self._pool.slab_bytes)
        self._residency = ResidencyMap(self._registry)
        self._scheduler = self._new_scheduler(prefetch_window=0)

        if torch.cuda.is_available():
            managed = {id(m) for m in self._layer_map.values()}
            for module in model.modules():
                if id(module) in managed:
                    continue
                for p in module.parameters(recurse=False):
                    p.data = p.data.to("cuda", dtype=dtype) if p.data.is_floating_point() else p.data.to("cuda")
                for bname, buf in module.named_buffers(recurse=False):
                    setattr(module, bname, buf.to("cuda", dtype=dtype) if buf.is_floating_point() else buf.to("cuda"))

        self._trace_order: list[str] = []
        self._trace_seen: set[str] = set()
        self._step = 0
        self._forward_started = False
        self._hook_handles: list = []
        self._mode = "trace"
        self._install_hooks(self._registry_order(), trace=True)
        _native.track(self, _native.CLOSE_RUNTIME, "shutdown")
        log.info("layer mode: tracing %d layers; pinned pool %d MB in %d MB slabs; prefetch_k=%d",
                 len(layers), self._config.pinned_pool_mb, self._config.pinned_slab_mb, prefetch_k)

    def _new_scheduler(self, prefetch_window: int) -> StagehandScheduler:
        return StagehandScheduler(
            registry=self._registry, residency=self._residency, transfer_engine=self._engine, budget=self._budget,
            policy=StaticLookaheadPolicy(prefetch_window=prefetch_window, eviction_cooldown_steps=0),
            guards=self._guards, telemetry=self._telemetry_inst, config=self._config,
            inference_mode=self._inference_mode,
        )

    def _registry_order(self) -> list[str]:
        return [e.block_id for e in self._registry.blocks_in_order() if e.module_ref() is not None]

    # ── hooks ────────────────────────────────────────────────────────

    def _install_hooks(self, order: list[str], trace: bool) -> None:
        for lid in order:
            module = self._layer_map.get(lid)
            if module is None:
                continue
            pre = self._make_trace_pre_hook(lid) if trace else self._make_scheduled_pre_hook(lid)
            self._hook_handles.append(module.register_forward_pre_hook(pre))
            self._hook_handles.append(module.register_forward_hook(self._make_post_hook(lid)))
            if trace and not self._inference_mode:
                self._install_backward(lid, module)
        if not trace and not self._inference_mode:
            for lid in reversed(order):
                module = self._layer_map.get(lid)
                if module is not None:
                    self._install_backward(lid, module)

    def _install_backward(self, lid: str, module: nn.Module) -> None:
        self._hook_handles.append(module.register_full_backward_pre_hook(self._make_bwd_pre_hook(lid)))
        self._hook_handles.append(module.register_full_backward_hook(self._make_bwd_post_hook(lid)))

    def _make_trace_pre_hook(self, layer_id: str):
        def hook(module: nn.Module, args: tuple) -> None:
            if self._trace_order and layer_id == self._trace_order[0] and self._forward_started:
                self._complete_trace()
                self._scheduler.before_block(layer_id)  # the new scheduled hook does not fire for this call
                return
            if layer_id not in self._trace_seen:
                self._trace_order.append(layer_id)
                self._trace_seen.add(layer_id)
            if not self._forward_started:
                self._scheduler.begin_step(self._step)
                self._forward_started = True
            self._scheduler.before_block(layer_id)
        return hook

    def _make_scheduled_pre_hook(self, layer_id: str):
        def hook(module: nn.Module, args: tuple) -> None:
            if layer_id == self._trace_order[0] and self._forward_started:
                self._record_pool_stats()
                self._scheduler.end_step()
                self._step += 1
                self._scheduler.begin_step(self._step)
            if not self._forward_started:
                self._scheduler.begin_step(self._step)
                self._forward_started = True
            self._scheduler.before_block(layer_id)
        return hook

    def _make_post_hook(self, layer_id: str):
        def hook(module: nn.Module, args: tuple, output: object) -> None:
            out = output if isinstance(output, torch.Tensor) else (
                output[0] if isinstance(output, (tuple, list)) and output and isinstance(output[0], torch.Tensor) else None)
            self._scheduler.after_block(layer_id, out)
        return hook

    def _make_bwd_pre_hook(self, layer_id: str):
        def hook(module: nn.Module, grad_output: tuple) -> None:
            self._scheduler.before_block(layer_id)
        return hook

    def _make_bwd_post_hook(self, layer_id: str):
        def hook(module: nn.Module, grad_input: tuple, grad_output: tuple) -> None:
            self._scheduler.after_block(layer_id)
        return hook

    # ── trace → scheduled ────────────────────────────────────────────

    def _complete_trace(self) -> None:
        self._record_pool_stats()
        self._scheduler.end_step()
        self._remove_hooks()
        old_scheduler = self._scheduler
        self._registry = BlockRegistry()
        self._registry.build_from_module_list([(lid, self._layer_map[lid]) for lid in self._trace_order], "layer", self._dtype)
        self._registry.validate(pool_capacity_bytes=self._pool.num_slabs * self._pool.slab_bytes)
        # A fresh residency map, as in the reference: layers loaded during the
        # trace are UNLOADED again and reload from their current parameters.
        self._residency = ResidencyMap(self._registry)
        self._scheduler = self._new_scheduler(prefetch_window=self._prefetch_k)
        self._scheduler._plans = old_scheduler._plans  # device plans stay valid across the rebuild
        self._install_hooks(list(self._trace_order), trace=False)
        self._step += 1
        self._scheduler.begin_step(self._step)
        self._forward_started = True
        self._mode = "scheduled"
        log.info("layer mode: traced %d layers in execution order; scheduling them with prefetch_k=%d",
                 len(self._trace_order), self._prefetch_k)

    def _remove_hooks(self) -> None:
        for h in self._hook_handles:
            h.remove()
        self._hook_handles.clear()

    def _record_pool_stats(self) -> None:
        st = self._pool.stats()
        self._telemetry_inst.record_pool_stats(free=int(st["free"]), in_use=int(st["in_use"]))
        self._telemetry_inst.record_vram(used_mb=self._budget.vram_used_mb(), reserved_mb=self._budget.vram_reserved_mb())

    # ── shutdown / properties ────────────────────────────────────────

    def shutdown(self) -> None:
        if self._mode == "shutdown":
            return
        self._remove_hooks()
        self._engine.shutdown()
        self._scheduler.close()
        self._pool.shutdown()
        self._telemetry_inst.close()
        self._mode = "shutdown"

    def shutdown_keep_pool(self) -> PinnedPool:
        if self._mode == "shutdown":
            raise RuntimeError("this layer runtime has been shut down")
        self._remove_hooks()
        self._engine.shutdown()
        self._scheduler.close()
        self._telemetry_inst.close()
        self._mode = "shutdown"
        return self._pool

    @property
    def telemetry(self) -> StagehandTelemetry:
        return self._telemetry_inst

    @property
    def stats(self) -> dict:
        return {"pool": self._pool.stats(),
                "telemetry": {"hit_rate": self._telemetry_inst.hit_rate(), "mean_stall_ms": self._telemetry_inst.mean_stall_ms()}}

    @property
    def traced(self) -> bool:
        return self._mode == "scheduled"

    @property
    def mode(self) -> str:
        return self._mode

    @property
    def num_layers(self) -> int:
        return len(self._all_layer_names)

    @property
    def trace_order(self) -> list[str]:
        return list(self._trace_order)

    @property
    def step(self) -> int:
        return self._step

    @property
    def config(self) -> StagehandConfig:
        return self._config

    @property
    def pool(self) -> PinnedPool:
        return self._pool

    @property
    def scheduler(self) -> StagehandScheduler:
        return self._scheduler

    @property
    def residency(self) -> ResidencyMap:
        return self._residency
