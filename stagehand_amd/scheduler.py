"""Block scheduler: prefetch window, eviction and the block load path.

Control decisions are those of src/stagehand/scheduler.py — the static
lookahead policy (:65-142), ``before_block``/``after_block`` (:773-850), the
prefetch window (:854-883), the load state walk (:885-951), eviction scoring
and protection (:1128-1182) and the eviction branches (:1184-1375) — and the
telemetry counters are incremented at the same points. What changed is the
load itself, on a GPU:

* a block's parameters are described as source pieces + an unpack plan
  (``stagehand_amd.staging``) instead of being cast / dequantised on the host;
* the native loader stages, copies and unpacks on its own thread and streams
  (``AsyncTransferEngine.submit_block_load``);
* ``before_block`` orders the compute stream after the load on the device
  (``wait_device``) instead of blocking the host in ``event.synchronize()``;
* module-backed blocks (the reference's synchronous pageable copy on the
  compute stream, :1033-1087) go through the same pinned-slab loader; the
  block is marked GPU_READY at once, as in the reference, and the compute
  stream waits for the data when the block is first used.

Without a GPU the scheduler runs the reference's CPU behaviour (host copies
and casts into CPU tensors); SquareQ dequantisation exists only on the device.
"""
from __future__ import annotations

import collections
import contextlib

import logging
import mmap
import os
import time
import warnings
from pathlib import Path
from typing import TYPE_CHECKING, Any, Protocol

import torch
from torch import nn

from stagehand_amd.fileio import FileCache, FileRange
from stagehand_amd.residency import BlockState
from stagehand_amd.staging import PlanCache, SourceBuilder, squareq_weight_tensors
from stagehand_amd.transfer import NativeEvent

if TYPE_CHECKING:
    from stagehand_amd.config import StagehandConfig
    from stagehand_amd.registry import BlockEntry, BlockRegistry, FileParamSpec
    from stagehand_amd.residency import ResidencyEntry, ResidencyMap
    from stagehand_amd.telemetry import StagehandTelemetry
    from stagehand_amd.transfer import AsyncTransferEngine, TransferHandle

__all__ = ["StaticLookaheadPolicy", "StagehandScheduler", "BudgetLike", "GuardsLike"]

log = logging.getLogger(__name__)
_STALL_LOGS_ENABLED = str(os.getenv("SERENITY_STAGEHAND_STALL_LOGS", "0")).strip().lower() in {"1", "true", "yes", "on"}

Layout = list[tuple[str, tuple[int, ...], torch.dtype, int, int]]


class BudgetLike(Protocol):
    def above_high_watermark(self) -> bool: ...
    def below_low_watermark(self) -> bool: ...


class GuardsLike(Protocol):
    def check_output(self, tensor: torch.Tensor, block_id: str, step: int) -> tuple[int, int]: ...


# ── policy ───────────────────────────────────────────────────────────────


class StaticLookaheadPolicy:
    """Prefetch the next ``prefetch_window`` blocks; evict by next-use distance × size."""

    def __init__(self, prefetch_window: int = 3, eviction_cooldown_steps: int = 2) -> None:
        self.prefetch_window = prefetch_window
        self.eviction_cooldown_steps = eviction_cooldown_steps

    def blocks_to_prefetch(self, cursor: int, total_blocks: int, residency_states: dict[str, str]) -> list[int]:
        return [cursor + k for k in range(1, self.prefetch_window + 1) if cursor + k < total_blocks]

    def score_for_eviction(self, block_id: str, current_cursor: int, entry_exec_order: int, total_blocks: int,
                           size_bytes: int) -> float:
        distance = (entry_exec_order - current_cursor) % total_blocks
        if distance == 0:
            distance = total_blocks  # just used / about to be used: farthest in wrap-around order
        return float(distance * size_bytes)

    def should_evict(self, last_used_step: int, current_step: int) -> bool:
        return current_step - last_used_step > self.eviction_cooldown_steps


# ── layout helpers (src/stagehand/scheduler.py:148-165, 328-346, 396-423) ──


def _build_param_layout(module: nn.Module, dtype: torch.dtype) -> Layout:
    layout: Layout = []
    offset = 0
    for name, param in module.named_parameters():
        numel = param.numel()
        layout.append((name, tuple(param.shape), dtype, offset, numel))
        offset += numel * dtype.itemsize
    return layout


def _get_param_data(module: nn.Module, dotted_name: str) -> torch.Tensor:
    owner = module
    parts = dotted_name.split(".")
    for part in parts[:-1]:
        owner = getattr(owner, part)
    return getattr(owner, parts[-1]).data


def _set_param_data(module: nn.Module, dotted_name: str, data: torch.Tensor) -> None:
    owner = module
    parts = dotted_name.split(".")
    for part in parts[:-1]:
        owner = getattr(owner, part)
    param = getattr(owner, parts[-1])
    try:
        param.data = data
    except RuntimeError:
        setattr(owner, parts[-1], nn.Parameter(data, requires_grad=param.requires_grad))


def _restore_params_from_tensor(module: nn.Module, flat_tensor: torch.Tensor, layout: Layout) -> None:
    """Point every parameter's ``.data`` at its view of the contiguous buffer."""
    flat = flat_tensor.view(torch.uint8) if flat_tensor.dtype != torch.uint8 else flat_tensor
    for name, shape, dtype, offset, numel in layout:
        nbytes = numel * dtype.itemsize
        _set_param_data(module, name, flat[offset:offset + nbytes].view(dtype).reshape(shape))


def _detach_params(module: nn.Module, layout: Layout) -> None:
    for name, _shape, dtype, _off, _numel in layout:
        _set_param_data(module, name, torch.empty(0, dtype=dtype))


def _runtime_dtype_on_host(value: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """A module-resident parameter of a file- or SquareQ-backed block, in the runtime dtype.

    Eviction saves such parameters back in the runtime dtype, so a parameter that
    starts out in another dtype (fp32 norm weights of a bf16 model) changes dtype
    after the block's first eviction. Casting it on the host at every load keeps
    the block's source layout, and so its pinned source image, the same from the
    first load on. The values are those of the device cast: torch's CPU
    conversion rounds to nearest even, as the unpack kernel does."""
    if value.dtype == dtype or not value.is_floating_point():
        return value
    return value.detach().to(device="cpu", dtype=dtype)


def _flatten_params_into_buffer(module: nn.Module, buffer: torch.Tensor, layout: Layout) -> None:
    """Host path (no GPU): ``region.copy_(param.to(dtype))`` per parameter (src/stagehand/scheduler.py:168-181)."""
    params = dict(module.named_parameters())
    for name, _shape, dtype, offset, numel in layout:
        region = buffer[offset:offset + numel * dtype.itemsize].view(dtype)
        region.copy_(params[name].data.to(dtype).reshape(-1))


# ── scheduler ────────────────────────────────────────────────────────────


class StagehandScheduler:
    def __init__(
        self,
        registry: BlockRegistry,
        residency: ResidencyMap,
        transfer_engine: AsyncTransferEngine,
        budget: BudgetLike,
        policy: StaticLookaheadPolicy,
        guards: GuardsLike | None,
        telemetry: StagehandTelemetry,
        config: StagehandConfig,
        inference_mode: bool = False,
    ) -> None:
        self._registry = registry
        self._residency = residency
        self._engine = transfer_engine
        self._budget = budget
        self._policy = policy
        self._guards = guards
        self._telemetry = telemetry
        self._config = config
        self._inference_mode = inference_mode
        self._has_cuda = torch.cuda.is_available()
        self._device = "cuda" if self._has_cuda else "cpu"

        self._current_step = 0
        self._cursor = 0
        self._backward_phase = False
        self._defer_backward_eviction = False
        self._ordered_blocks: list[BlockEntry] = []
        self._total_blocks = 0
        self._order_to_id: dict[int, str] = {}
        self.refresh_registry_snapshot()

        self._pending_handles: dict[str, TransferHandle] = {}
        self._conductor_adapter = None
        self._squareq_adapter = None
        self._eriquant_adapter = None
        self._file_maps: dict[str, tuple[Any, mmap.mmap, memoryview]] = {}
        self._file_tensor_views: dict[tuple, torch.Tensor] = {}
        reader = getattr(config, "file_reader", "mmap")
        if reader not in ("mmap", "pread", "direct"):
            raise ValueError(f"file_reader must be 'mmap', 'pread' or 'direct', got {reader!r}")
        if getattr(config, "save_back_fence", "last_use") not in ("last_use", "whole_queue"):
            raise ValueError(f"save_back_fence must be 'last_use' or 'whole_queue', got {config.save_back_fence!r}")
        # native weight-file reads (file_reader "pread"/"direct"): the device path only
        self._file_reader = reader if self._has_cuda else "mmap"
        self._weight_files = FileCache()
        self._v2_locations: dict[str, dict] = {}  # SquareQ V2 file → layer → tensor locations
        self._v2_zp_nonzero: dict[tuple, bool] = {}
        self._squareq_layers: dict[str, dict[str, Any]] = {}
        self._module_param_caches: dict[str, dict[str, torch.Tensor]] = {}
        self._plans = PlanCache()
        # block → event of the asynchronous D2H that moved its module parameters
        # to host memory at eviction; waited for before those tensors are read
        self._d2h_fences: dict[str, Any] = {}
        # block → {param name: host tensor} kept for frozen module parameters while
        # the block is resident (config.frozen_host_copies)
        self._host_copies: dict[str, dict[str, torch.Tensor]] = {}
        # block → pinned host buffer in the block's layout, the target of its whole-block save-backs
        self._host_homes: dict[str, torch.Tensor] = {}
        # save-backs of changed chunks (config.save_back_changed_chunks): per block, the device
        # buffer of its chunk digests, the (digests, bytes, chunk bytes) its last load from the
        # home buffer wrote, and the pinned byte-per-chunk flags its save-backs compare into
        self._digest_bufs: dict[str, torch.Tensor] = {}
        self._load_digests: dict[str, tuple[torch.Tensor, int, int]] = {}
        self._changed_flags: dict[str, torch.Tensor] = {}
        # events recorded on the compute stream after each block (config.max_run_ahead_blocks)
        self._done_marks: collections.deque = collections.deque()
        # save-back fences (_save_back_fence): per module-backed block, an event after its last
        # hook or gradient accumulation; an event where the step began; the blocks' parameter
        # version counters then; the gradient-accumulation hooks that record those events
        self._last_use: dict[str, Any] = {}
        self._step_mark: Any = None
        self._step_versions: dict[str, tuple[int, ...]] = {}
        self._in_step = False
        self._grad_hooks: list = []
        # blocks loaded since their last after_block: the load (and the gradients moved to the
        # device with it) may still be writing them, so their save-backs wait for the whole queue
        self._unsettled: set[str] = set()
        # save-back fences taken, by kind (telemetry): the block's last use, or the whole queue and why
        self.fence_kinds: collections.Counter = collections.Counter()
        # device memory that an eviction gave up is left out of the budget while the
        # save-back copy still holds it (the reference's synchronous copy frees it at once)
        count_as_released = getattr(budget, "count_as_released", None)
        releasing = getattr(transfer_engine, "releasing_bytes", None)
        if callable(count_as_released) and callable(releasing):
            count_as_released(releasing)

    # ── step lifecycle ───────────────────────────────────────────────

    def refresh_registry_snapshot(self) -> None:
        self._ordered_blocks = self._registry.blocks_in_order()
        self._total_blocks = len(self._ordered_blocks)
        self._order_to_id = {e.exec_order: e.block_id for e in self._ordered_blocks}

    def begin_step(self, step: int) -> None:
        self._current_step = step
        self._cursor = 0
        self._backward_phase = False
        self._telemetry.begin_step(step)
        self._mark_step_begin()

    def end_step(self) -> None:
        self._remove_grad_hooks()
        self._backward_phase = False
        self._sync_d2h_fences()
        self._engine.reap()
        self._reconcile_file_backed_grads()
        self._telemetry.end_step()

    def enter_backward_phase(self) -> None:
        self._backward_phase = True

    def exit_backward_phase(self) -> None:
        self._backward_phase = False

    @property
    def in_backward_phase(self) -> bool:
        return self._backward_phase

    def set_defer_backward_eviction(self, enabled: bool) -> None:
        self._defer_backward_eviction = enabled

    def _sync_d2h_fences(self, block_id: str | None = None) -> None:
        """Host values of evicted module parameters are final once their D2H event completes."""
        ids = list(self._d2h_fences) if block_id is None else ([block_id] if block_id in self._d2h_fences else [])
        for bid in ids:
            ev = self._d2h_fences.pop(bid)
            if ev is not None:
                with self._host_wait("d2h_fence"):
                    ev.synchronize()

    # ── save-back fences ─────────────────────────────────────────────

    def _module_backed_modules(self):
        for entry in self._ordered_blocks:
            if entry.file_backed or entry.squareq_backed or entry.eriquant_backed:
                continue
            module = entry.module_ref()
            if module is not None:
                yield entry.block_id, module

    def _mark_step_begin(self) -> None:
        """Records where the step began (after the previous step's optimizer) and the parameter
        version counters of the module-backed blocks then, and hooks gradient accumulation of
        their trainable parameters until end_step (for the save-back fences)."""
        self._remove_grad_hooks()
        record = getattr(self._engine, "record_event", None)
        # inference evicts without save-backs (the eviction loop), so it needs none of this
        self._step_mark = record() if self._has_cuda and callable(record) and not self._inference_mode else None
        self._in_step = self._step_mark is not None
        if not self._in_step:
            return
        self._step_versions = {}
        for block_id, module in self._module_backed_modules():
            params = list(module.parameters())
            self._step_versions[block_id] = tuple(p._version for p in params)
            hook = self._grad_hook_for(block_id)
            self._grad_hooks.extend(p.register_post_accumulate_grad_hook(hook) for p in params if p.requires_grad)

    def _grad_hook_for(self, block_id: str):
        def hook(_param: torch.Tensor) -> None:
            self._record_last_use(block_id)
        return hook

    def _record_last_use(self, block_id: str) -> None:
        if self._in_step:
            self._last_use[block_id] = self._engine.record_event()

    def _save_back_fence(self, block_id: str, module: nn.Module | None) -> list | None:
        """What a save-back of the block's parameters and gradients waits for before it starts:
        a list of events, or None for everything queued on the current stream so far (the
        reference's synchronous copy).

        Inside a step, the work queued since the block's last hook and its last gradient
        accumulation belongs to other blocks: it reads their parameters, not this block's. The
        optimizer and other work between steps is before the step's start. So the copy needs only
        those events, and the save-back engine need not wait for compute queued far ahead of it
        (the host runs ahead of the device by up to max_run_ahead_blocks blocks). The whole queue
        is waited for when a parameter changed in place since the step began (its version counter
        moved) and when the block was loaded again after its last hook (the load, and gradients
        moved to the device with it, write it; the eviction has ordered the current stream after
        the load). Writes through ``param.data`` do not move the counter and are not seen here;
        ``StagehandConfig.save_back_fence="whole_queue"`` makes every save-back wait for the whole
        queue instead."""
        if getattr(self._config, "save_back_fence", "last_use") == "whole_queue":
            self.fence_kinds["whole_queue_configured"] += 1
            return None
        if not self._in_step or module is None:
            self.fence_kinds["whole_queue_outside_step"] += 1
            return None
        if block_id in self._unsettled:
            self.fence_kinds["whole_queue_loaded_since_last_use"] += 1
            return None
        versions = self._step_versions.get(block_id)
        if versions is None or versions != tuple(p._version for p in module.parameters()):
            self.fence_kinds["whole_queue_changed_in_place"] += 1
            return None
        last = self._last_use.get(block_id)
        self.fence_kinds["last_use"] += 1
        return [self._step_mark] if last is None else [last, self._step_mark]

    def _remove_grad_hooks(self) -> None:
        for h in self._grad_hooks:
            h.remove()
        self._grad_hooks.clear()
        self._last_use.clear()
        self._step_mark = None
        self._in_step = False

    def _host_wait(self, kind: str):
        """The engine's host-wait accounting (a no-op context for engines without it)."""
        wait = getattr(self._engine, "host_wait", None)
        return wait(kind) if wait is not None else contextlib.nullcontext()

    def _save_params_to_host(self, block_id: str, module: nn.Module, names: list[str], with_grads: bool = False) -> None:
        """``param.data = param.data.to("cpu").clone()`` for ``names`` (and grads), without a host sync.

        The reference does this synchronously at eviction (src/stagehand/scheduler.py:1216-1231,
        :1348-1366), which stalls the host on the whole device queue once per block. Here the
        copies run on the copy stream into pinned host tensors; the block's fence is waited
        for before the tensors are read again (next staging, end of step, shutdown).
        """
        srcs, targets = [], []
        for name in names:
            data = _get_param_data(module, name)
            if data.device.type != "cpu":
                srcs.append(data)
                targets.append(("data", name))
        if with_grads:
            for name, param in module.named_parameters():
                if param.grad is not None and param.grad.device.type != "cpu":
                    srcs.append(param.grad)
                    targets.append(("grad", name))
        if not srcs:
            return
        # a parameter viewing the block buffer is copied out of it on the device first, so the
        # buffer is not held until the save-back completes (it is freed when the block is dropped)
        views = [t.untyped_storage().nbytes() > t.numel() * t.element_size() for t in srcs]
        srcs = [t.clone() if v else t for t, v in zip(srcs, views)]
        # the clones are queued on the current stream now: then the copy waits for the whole queue
        after = None if any(views) else self._save_back_fence(block_id, module)
        outs, ev = self._engine.d2h_async(srcs, after=after)
        params = dict(module.named_parameters())
        for (what, name), out in zip(targets, outs):
            if what == "data":
                _set_param_data(module, name, out)
            else:
                params[name].grad = out
        if ev is not None:
            prev = self._d2h_fences.get(block_id)
            self._d2h_fences[block_id] = ev if prev is None else ev  # later event covers earlier copies on the stream

    def _save_block_home(self, block_id: str, module: nn.Module, res_entry: ResidencyEntry, names: list[str]) -> bool:
        """Save-back of a whole module-backed block in one copy into its pinned home buffer.

        Used when every parameter is copied back and is still its view of the block's device
        buffer: that buffer is then the block's bytes in the layout, so one D2H copies it into
        a pinned host buffer kept for the block (allocated at its first eviction, reused after)
        and the parameters become views of it. The next load finds pinned pieces in the
        layout and copies them back in one DMA. When that load took chunk digests
        (``_home_load_digest``), only the chunks changed on the device since are copied.
        Returns False to take the per-parameter path.
        """
        layout, gpu = res_entry.param_layout, res_entry.gpu_tensor
        if not self._has_cuda or layout is None or gpu is None or set(names) != {n for n, *_ in layout}:
            return False
        base = gpu.view(torch.uint8)
        bptr = base.data_ptr()
        end = 0
        for name, _shape, dtype, off, numel in layout:
            d = _get_param_data(module, name)
            if (d.device != gpu.device or d.dtype != dtype or d.numel() != numel or not d.is_contiguous()
                    or d.data_ptr() != bptr + off):
                return False
            end = max(end, off + numel * dtype.itemsize)
        home = self._host_homes.get(block_id)
        fresh = home is None or home.numel() < end
        if fresh:
            home = torch.empty(end, dtype=torch.uint8, pin_memory=True)
            self._host_homes[block_id] = home
        after = self._save_back_fence(block_id, module)
        loaded = self._load_digests.pop(block_id, None)
        ev = None
        if not fresh and loaded is not None and loaded[1] == end:
            # the block was loaded from this home buffer and its digests taken then: copy back the
            # chunks that changed on the device since
            chunk = loaded[2]
            n_chunks = -(-end // chunk)
            flags = self._changed_flags.get(block_id)
            if flags is None or flags.numel() < n_chunks:
                flags = torch.zeros(n_chunks, dtype=torch.uint8, pin_memory=True)
                self._changed_flags[block_id] = flags
            ev = self._engine.d2h_changed(base[:end], home[:end], chunk, loaded[0], flags, after=after)
        if ev is None:
            ev = self._engine.d2h_into(base[:end], home[:end], after=after)
        _restore_params_from_tensor(module, home, layout)
        if ev is not None:
            self._d2h_fences[block_id] = ev
        return True

    def _chunk_bytes(self) -> int:
        return int(getattr(self._config, "save_back_chunk_bytes", 1 << 18))

    def _home_load_digest(self, block_id: str, module: nn.Module, layout) -> tuple[torch.Tensor, int, int] | None:
        """Where a module-backed load writes its chunk digests, or None for no digests.

        Digests are taken only when the load's source is exactly the block's home buffer (every
        parameter its view at its layout offset, in the layout's dtype, as a whole-block
        save-back left them): the device then starts out with the home buffer's bytes, so its
        next save-back may skip the chunks whose digests have not changed. A source built any
        other way (parameters replaced on the host, a cast on load) takes a full save-back."""
        if not (self._has_cuda and getattr(self._config, "save_back_changed_chunks", False)
                and getattr(self._config, "save_back_engine", "sdma") == "sdma"):
            return None
        home = self._host_homes.get(block_id)
        if home is None or layout is None:
            return None
        hptr, end = home.data_ptr(), 0
        for name, _shape, dtype, off, numel in layout:
            d = _get_param_data(module, name)
            if (d.device.type != "cpu" or d.dtype != dtype or d.numel() != numel or not d.is_contiguous()
                    or d.data_ptr() != hptr + off):
                return None
            end = max(end, off + numel * dtype.itemsize)
        if end == 0 or end > home.numel():
            return None
        chunk = self._chunk_bytes()
        n_words = 2 * -(-end // chunk)
        dig = self._digest_bufs.get(block_id)
        if dig is None or dig.numel() < n_words:
            dig = torch.empty(n_words, dtype=torch.int64, device="cuda")  # two uint64 sums per chunk
            self._digest_bufs[block_id] = dig
        return dig, end, chunk

    def _release_with_save_back(self, block_id: str, res_entry: ResidencyEntry, fence_before: Any) -> None:
        """The block's device buffer, about to be dropped, stays held by the whole-block save-back
        just queued for it (its fence changed): count it as released for the budget from now on.
        Per-parameter save-backs copy views of the buffer out first and do not hold it."""
        fence = self._d2h_fences.get(block_id)
        gpu = res_entry.gpu_tensor
        if fence is None or fence is fence_before or gpu is None or not hasattr(self._engine, "release_with_copy"):
            return
        self._engine.release_with_copy(fence, gpu.untyped_storage().nbytes())

    def _take_host_copies(self, block_id: str, module: nn.Module, names: list[str]) -> list[str]:
        """Points frozen parameters kept with a host copy back at it; returns the names still to copy back."""
        kept = self._host_copies.pop(block_id, None)
        if not kept:
            return names
        params = dict(module.named_parameters())
        rest = []
        for name in names:
            host = kept.get(name)
            if host is not None and name in params and not params[name].requires_grad:
                _set_param_data(module, name, host)
            else:
                rest.append(name)
        return rest

    def _reconcile_file_backed_grads(self) -> None:
        for entry in self._ordered_blocks:
            if not entry.file_backed:
                continue
            module = entry.module_ref()
            mutable = set(entry.module_param_names)
            if module is None or not mutable:
                continue
            for name, param in module.named_parameters():
                if name in mutable and param.device.type == "cpu" and param.grad is not None \
                        and param.grad.device.type != "cpu":
                    param.grad = param.grad.to("cpu", non_blocking=True)

    # ── sources ──────────────────────────────────────────────────────

    def _get_file_view(self, source_path: str) -> memoryview:
        key = str(Path(source_path).expanduser())
        hit = self._file_maps.get(key)
        if hit is not None:
            return hit[2]
        fh = Path(key).open("rb")
        mm = mmap.mmap(fh.fileno(), length=0, access=mmap.ACCESS_READ)
        view = memoryview(mm)
        self._file_maps[key] = (fh, mm, view)
        return view

    def _get_file_tensor_view(self, source_path: str, spec: FileParamSpec, file_view: memoryview | None = None) -> torch.Tensor:
        path = str(Path(source_path).expanduser())
        key = (path, int(spec.file_offset), int(spec.source_nbytes), spec.source_dtype, spec.source_shape)
        hit = self._file_tensor_views.get(key)
        if hit is not None:
            return hit
        view = file_view if file_view is not None else self._get_file_view(path)
        region = view[int(spec.file_offset):int(spec.file_offset) + int(spec.source_nbytes)]
        with warnings.catch_warnings():
            warnings.simplefilter("ignore", UserWarning)  # read-only mmap: never written through
            t = torch.frombuffer(region, dtype=spec.source_dtype).reshape(spec.source_shape)
        self._file_tensor_views[key] = t
        return t

    def _get_squareq_layers(self, source_path: str) -> dict[str, Any]:
        key = str(Path(source_path).expanduser())
        hit = self._squareq_layers.get(key)
        if hit is not None:
            return hit
        payload = torch.load(key, map_location="cpu", weights_only=True, mmap=True)
        if not isinstance(payload, dict):
            raise ValueError(f"Invalid SquareQ slab payload at {key}")
        layers = payload.get("layers")
        if not isinstance(layers, dict):
            raise ValueError(f"SquareQ slab missing 'layers' map at {key}")
        self._squareq_layers[key] = layers
        return layers

    def _get_squareq_v2_layers(self, source_path: str) -> dict[str, Any]:
        """V2: safetensors slab + ``<stem>.manifest.json``; tensors are zero-copy views of the mapped file."""
        from stagehand_amd.squareq_v2 import read_v2_layers

        key = str(Path(source_path).expanduser())
        hit = self._squareq_layers.get(key)
        if hit is not None:
            return hit
        layers = read_v2_layers(key, str(Path(key).with_suffix(".manifest.json")), self._get_file_view(key))
        self._squareq_layers[key] = layers
        return layers

    def close(self) -> None:
        self._sync_d2h_fences()
        self._remove_grad_hooks()
        self._file_tensor_views.clear()
        for fh, mm, view in self._file_maps.values():
            for fn in (view.release, mm.close, fh.close):
                try:
                    fn()
                except Exception:
                    pass
        self._file_maps.clear()
        self._weight_files.close()
        self._host_homes.clear()
        self._digest_bufs.clear()
        self._load_digests.clear()
        self._changed_flags.clear()
        self._v2_locations.clear()
        self._squareq_layers.clear()
        self._module_param_caches.clear()
        self._plans.clear()

    # ── external bandwidth adapters (not part of this build's path) ──

    def set_conductor_adapter(self, adapter: Any) -> None:
        self._conductor_adapter = adapter

    def set_squareq_adapter(self, adapter: Any) -> None:
        self._squareq_adapter = adapter

    def set_eriquant_adapter(self, adapter: Any) -> None:
        self._eriquant_adapter = adapter

    # ── per-block hooks ──────────────────────────────────────────────

    def _run_ahead_limit(self) -> int:
        """``max_run_ahead_blocks`` in training, ``max_run_ahead_blocks_inference`` in inference."""
        if self._inference_mode:
            return int(getattr(self._config, "max_run_ahead_blocks_inference", 0))
        return int(getattr(self._config, "max_run_ahead_blocks", 0))

    def _bound_run_ahead(self) -> None:
        """Host wait for the compute of the block ``_run_ahead_limit()`` back."""
        limit = self._run_ahead_limit()
        while limit > 0 and len(self._done_marks) >= limit:
            mark = self._done_marks.popleft()
            with self._host_wait("run_ahead"):
                mark.synchronize()

    def _mark_block_done(self) -> None:
        if self._has_cuda and self._run_ahead_limit() > 0:
            ev = NativeEvent()
            ev.record(torch.cuda.current_stream().cuda_stream)
            self._done_marks.append(ev)

    def before_block(self, block_id: str) -> None:
        self._bound_run_ahead()
        self._engine._reap_d2h()  # release device buffers whose save-back copies finished
        state = self._residency.get_state(block_id)
        if state == BlockState.GPU_READY:
            self._telemetry.record_prefetch_hit()
            self._await_pending_load(block_id)
        elif state == BlockState.PREFETCHING:
            t0 = time.monotonic()
            self._complete_prefetch(block_id)
            stall_ms = (time.monotonic() - t0) * 1000.0
            self._telemetry.record_stall(stall_ms)
            self._telemetry.record_prefetch_miss()
            log.debug("Stall on block %s: %.2f ms", block_id, stall_ms)
        else:
            t0 = time.monotonic()
            self._load_block_to_gpu(block_id)
            if self._residency.get_state(block_id) == BlockState.PREFETCHING:
                self._complete_prefetch(block_id)
            else:
                self._await_pending_load(block_id)
            stall_ms = (time.monotonic() - t0) * 1000.0
            self._telemetry.record_stall(stall_ms)
            self._telemetry.record_prefetch_miss()
            if _STALL_LOGS_ENABLED:
                log.warning("Hard stall on block %s (was %s): %.2f ms", block_id, state.value, stall_ms)

        self._residency.increment_ref(block_id)
        entry = self._residency.get_entry(block_id)
        entry.last_used_step = self._current_step
        if self._has_cuda and entry.gpu_tensor is not None:
            # block buffers come from the loader stream's pool (AsyncTransferEngine.alloc_device):
            # register the compute stream's use so the memory is not reused before it has run
            entry.gpu_tensor.record_stream(torch.cuda.current_stream())
        self._engine.mark_compute(block_id, start=True)
        self._cursor += 1
        if self._budget.above_high_watermark():
            self._run_eviction(ignore_cooldown=True)
        self._prefetch_ahead()
        if self._budget.above_high_watermark():
            self._run_eviction(ignore_cooldown=True)

    def after_block(self, block_id: str, output: torch.Tensor | None = None) -> None:
        self._engine.mark_compute(block_id, start=False)
        # the compute stream waited for the block's load before this block ran
        self._unsettled.discard(block_id)
        if self._in_step and block_id in self._step_versions:
            self._record_last_use(block_id)
        self._mark_block_done()
        self._residency.decrement_ref(block_id)
        self._residency.get_entry(block_id).last_used_step = self._current_step
        if self._guards is not None and output is not None and self._config.nan_inf_check:
            nan_count, inf_count = self._guards.check_output(output, block_id, self._current_step)
            if nan_count > 0 or inf_count > 0:
                self._telemetry.record_nan_inf(nan_count, inf_count)
        if self._budget.above_high_watermark() and not (self._backward_phase and self._defer_backward_eviction):
            self._run_eviction(ignore_cooldown=True)

    def _complete_prefetch(self, block_id: str) -> None:
        """PREFETCHING → GPU_READY: order the compute stream after the load, restore views."""
        handle = self._pending_handles.pop(block_id, None)
        if handle is not None:
            self._engine.wait_device(handle)
            self._residency.get_entry(block_id).load = None
        self._finalize_gpu_load(block_id)

    def _await_pending_load(self, block_id: str) -> None:
        entry = self._residency.get_entry(block_id)
        if entry.load is not None:
            self._engine.wait_device(entry.load)
            entry.load = None

    # ── prefetch ─────────────────────────────────────────────────────

    def _prefetch_ahead(self) -> None:
        states: dict[str, str] = {}
        if type(self._policy) is not StaticLookaheadPolicy:  # the built-in policy never reads the state map
            states = {e.block_id: self._residency.get_state(e.block_id).value for e in self._ordered_blocks}
        for idx in self._policy.blocks_to_prefetch(self._cursor - 1, self._total_blocks, states):
            if idx >= self._total_blocks:
                break
            block_id = self._ordered_blocks[idx].block_id
            if self._residency.get_state(block_id) in (BlockState.GPU_READY, BlockState.PREFETCHING):
                continue
            if not self._budget.can_prefetch():
                break
            self._load_block_to_gpu(block_id, speculative=True)

    def _load_block_to_gpu(self, block_id: str, speculative: bool = False) -> None:
        state = self._residency.get_state(block_id)
        if state in (BlockState.GPU_READY, BlockState.PREFETCHING):
            return
        block_entry = self._registry.get(block_id)
        res_entry = self._residency.get_entry(block_id)

        if block_entry.eriquant_backed:
            if self._eriquant_adapter is None:
                log.error("Block %r is eriquant-backed but no adapter set — skipping", block_id)
                return
            if state == BlockState.UNLOADED:
                self._eriquant_adapter.on_prefetch(block_id, self._device)
                for s in (BlockState.HOST_STAGED, BlockState.PREFETCHING, BlockState.GPU_READY):
                    self._residency.transition(block_id, s)
                self._telemetry.record_h2d(block_entry.size_bytes)
            return

        module_backed = not block_entry.file_backed and not block_entry.squareq_backed
        if module_backed and state == BlockState.UNLOADED:
            self._load_module_backed_direct(block_id, block_entry, res_entry)
            return

        if state == BlockState.UNLOADED:
            res_entry.host_slab = self._stage_block_to_host(block_entry, res_entry)
            state = self._residency.get_state(block_id)

        if state == BlockState.HOST_STAGED:
            if res_entry.gpu_tensor is None:
                numel = block_entry.size_bytes // block_entry.dtype.itemsize
                res_entry.gpu_tensor = (self._engine.alloc_device(numel, block_entry.dtype) if self._has_cuda else
                                        torch.empty(numel, dtype=block_entry.dtype, device=self._device))
                fresh = True
            else:
                fresh = False
            staged = res_entry.host_slab
            if self._has_cuda:
                handle = self._engine.submit_block_load(block_id, staged, res_entry.gpu_tensor.view(torch.uint8),
                                                        dest_on_loader_stream=fresh)
                res_entry.host_slab = None  # the loader owns slab staging and release
            else:
                handle = self._engine.submit_h2d(block_id, staged, res_entry.gpu_tensor)
            self._pending_handles[block_id] = handle
            self._unsettled.add(block_id)
            self._residency.transition(block_id, BlockState.PREFETCHING)
            self._telemetry.record_h2d(block_entry.size_bytes)

    def _stage_block_to_host(self, block_entry: BlockEntry, res_entry: ResidencyEntry):
        """UNLOADED → HOST_STAGED. On a GPU: returns the block's BlockSource (the
        loader fills a pinned slab from it). Without one: a filled pool slab,
        as in src/stagehand/scheduler.py:953-1031."""
        self._sync_d2h_fences(block_entry.block_id)
        module = block_entry.module_ref()
        if module is None:
            res_entry.param_layout = None
            staged = self._zero_source(block_entry)
        elif block_entry.squareq_backed or block_entry.file_backed:
            layout = list(block_entry.param_layout)
            res_entry.param_layout = layout
            staged = self._build_source(block_entry, module, layout)
        elif any(True for _ in module.parameters()):
            layout = _build_param_layout(module, block_entry.dtype)
            res_entry.param_layout = layout
            staged = self._build_module_source(block_entry, module, layout)
        else:
            res_entry.param_layout = None
            staged = self._zero_source(block_entry)
        self._residency.transition(block_entry.block_id, BlockState.HOST_STAGED)
        return staged

    # ── source building ──────────────────────────────────────────────

    def _zero_source(self, block_entry: BlockEntry):
        if self._has_cuda:
            b = SourceBuilder(block_entry.dtype, block_entry.size_bytes)
            b.add_zero(0, block_entry.size_bytes)
            return b.finish()[0]
        slab = self._engine._pool.acquire(block_entry.size_bytes)
        slab.buffer[:] = 0
        return slab

    def _finish_source(self, block_id: str, builder: SourceBuilder):
        source, descs = builder.finish()
        if descs is not None:
            source.plan = self._plans.get(block_id, descs)
        return source

    def _build_module_source(self, block_entry: BlockEntry, module: nn.Module, layout: Layout):
        if not self._has_cuda:
            slab = self._engine._pool.acquire(block_entry.size_bytes)
            _flatten_params_into_buffer(module, slab.buffer, layout)
            return slab
        params = dict(module.named_parameters())
        b = SourceBuilder(block_entry.dtype, block_entry.size_bytes)
        for name, _shape, _dtype, offset, _numel in layout:
            b.add_param(offset, params[name].data, mutable=True)
        source = self._finish_source(block_entry.block_id, b)
        source.key = None  # every byte is a live module parameter: nothing to keep pinned
        return source

    def _build_source(self, block_entry: BlockEntry, module: nn.Module, layout: Layout):
        if not self._has_cuda:
            slab = self._engine._pool.acquire(block_entry.size_bytes)
            if block_entry.squareq_backed:
                self._fill_squareq_host(block_entry, module, layout, slab.buffer)
            else:
                self._fill_file_backed_host(block_entry, module, layout, slab.buffer)
            return slab
        builder = SourceBuilder(block_entry.dtype, block_entry.size_bytes)
        if block_entry.squareq_backed:
            self._add_squareq_regions(block_entry, module, layout, builder)
        else:
            self._add_file_regions(block_entry, module, layout, builder)
        return self._finish_source(block_entry.block_id, builder)

    def _module_value(self, block_id: str, params: dict, name: str, numel: int,
                      cache: dict[str, torch.Tensor] | None) -> torch.Tensor | None:
        param = params.get(name)
        if param is not None and param.data.numel() == numel:
            if cache is not None and name not in cache:
                cache[name] = param.data.detach().cpu()
            return param.data
        if cache is not None and name in cache:
            return cache[name]
        return None

    def _add_file_regions(self, block_entry: BlockEntry, module: nn.Module, layout: Layout, b: SourceBuilder) -> None:
        """Safetensors-backed block (src/stagehand/scheduler.py:184-241)."""
        params = dict(module.named_parameters())
        specs = {s.param_name: s for s in block_entry.file_param_specs}
        mutable = set(block_entry.module_param_names)
        sharded = block_entry.source_format == "safetensors_sharded"
        native = self._file_reader != "mmap"
        for name, _shape, dtype, offset, numel in layout:
            spec = specs.get(name)
            if spec is not None:
                path = spec.file_path if (spec.file_path and sharded) else str(block_entry.source_path)
                if native:
                    wf = self._weight_files.get(str(Path(path).expanduser()), self._file_reader == "direct")
                    fr = FileRange(wf, int(spec.file_offset), int(spec.source_nbytes))
                    if b.add_file_param(offset, fr, spec.source_dtype,
                                        int(spec.source_nbytes) // spec.source_dtype.itemsize):
                        continue
                view = self._get_file_view(path) if (spec.file_path and sharded) else self._get_file_view(
                    str(block_entry.source_path))
                b.add_param(offset, self._get_file_tensor_view(path, spec, view))
                continue
            if name in mutable and name in params and params[name].data.numel() == numel:
                b.add_param(offset, _runtime_dtype_on_host(params[name].data, dtype), mutable=True)
                continue
            b.add_zero(offset, numel * dtype.itemsize)

    def _fill_file_backed_host(self, block_entry: BlockEntry, module: nn.Module, layout: Layout, buffer: torch.Tensor) -> None:
        params = dict(module.named_parameters())
        specs = {s.param_name: s for s in block_entry.file_param_specs}
        mutable = set(block_entry.module_param_names)
        sharded = block_entry.source_format == "safetensors_sharded"
        for name, _shape, dtype, offset, numel in layout:
            region = buffer[offset:offset + numel * dtype.itemsize]
            spec = specs.get(name)
            if spec is not None:
                path = spec.file_path if (spec.file_path and sharded) else str(block_entry.source_path)
                region.view(dtype).copy_(self._get_file_tensor_view(path, spec).reshape(-1))
            elif name in mutable and name in params and params[name].data.numel() == numel:
                region.view(dtype).copy_(params[name].data.to(dtype).reshape(-1))
            else:
                region.zero_()

    def _squareq_actions(self, block_entry: BlockEntry, module: nn.Module, layout: Layout, native_v2: bool):
        """The branch walk of src/stagehand/scheduler.py:243-325 for a SquareQ-backed block.

        Yields ``(offset, nbytes, dtype, action, payload)`` per layout entry in layout order:
        ``"dequant"`` with ``(q2d[:out], in_flat, scale, zero_point)``; ``"param"`` with the host
        tensor to cast into the region (a bias, or a module parameter / its cached copy);
        ``"zero"``; or ``"v2file"`` with ``(path, spec, shape, numel)`` for a V2 tensor that the
        native reader may take as file ranges (the caller falls back to the tensor branches by
        sending the entry back with ``generator.send(False)``)."""
        params = dict(module.named_parameters())
        specs = {s.param_name: s for s in block_entry.squareq_param_specs}
        mutable = set(block_entry.module_param_names)
        path = str(block_entry.source_path)
        v2 = block_entry.source_format == "squareq_v2"
        loaded: list[dict] = []

        def layers() -> dict[str, Any]:  # host views, only when a region needs them
            if not loaded:
                loaded.append(self._get_squareq_v2_layers(path) if v2 else self._get_squareq_layers(path))
            return loaded[0]

        cache = self._module_param_caches.setdefault(block_entry.block_id, {})
        for name, shape, dtype, offset, numel in layout:
            nbytes = numel * dtype.itemsize
            spec = specs.get(name)
            if spec is not None and native_v2:
                taken = yield offset, nbytes, dtype, "v2file", (path, spec, shape, numel)
                if taken:
                    continue
            if spec is not None:
                layer = layers().get(spec.layer_name)
                if isinstance(layer, dict):
                    if spec.kind == "weight":
                        tensors = squareq_weight_tensors(layer)
                        if tensors is not None:
                            q, s, z = tensors
                            out_dim = int(shape[0]) if len(shape) else 0
                            in_flat = numel // max(out_dim, 1) if out_dim else 0
                            if len(shape) == 0 or out_dim <= 0 or in_flat <= 0:
                                yield offset, nbytes, dtype, "zero", None
                                continue
                            q2d = q.reshape(int(q.shape[0]), -1)
                            sv, zv = s.reshape(-1), z.reshape(-1)
                            if sv[:out_dim].numel() != out_dim or zv[:out_dim].numel() != out_dim:
                                yield offset, nbytes, dtype, "zero", None
                                continue
                            if q2d.shape[0] < out_dim or q2d.shape[1] < in_flat:
                                raise ValueError(f"SquareQ layer {spec.layer_name!r}: qweight {tuple(q.shape)} "
                                                 f"is smaller than {out_dim}x{in_flat}")
                            yield offset, nbytes, dtype, "dequant", (q2d[:out_dim], in_flat, sv, zv)
                            continue
                    elif spec.kind == "bias":
                        bias = layer.get("bias")
                        if isinstance(bias, torch.Tensor):
                            yield offset, nbytes, dtype, "param", bias
                        else:
                            yield offset, nbytes, dtype, "zero", None
                        continue
            if name in mutable and name in params:
                value = self._module_value(block_entry.block_id, params, name, numel, cache)
                if value is not None:
                    yield offset, nbytes, dtype, "module", value
                    continue
            yield offset, nbytes, dtype, "zero", None

    def _add_squareq_regions(self, block_entry: BlockEntry, module: nn.Module, layout: Layout, b: SourceBuilder) -> None:
        """SquareQ-backed block on the device: each branch becomes a region of the block source."""
        native = block_entry.source_format == "squareq_v2" and self._file_reader != "mmap"
        walk = self._squareq_actions(block_entry, module, layout, native)
        item = next(walk, None)
        while item is not None:
            offset, nbytes, dtype, action, payload = item
            reply = None
            if action == "v2file":
                reply = self._add_v2_file_region(b, *payload, offset)
            elif action == "dequant":
                q2d, in_flat, sv, zv = payload
                b.add_dequant(offset, q2d, in_flat, sv, zv)
            elif action == "param":
                b.add_param(offset, payload)
            elif action == "module":
                b.add_param(offset, _runtime_dtype_on_host(payload, dtype), mutable=True)
            else:
                b.add_zero(offset, nbytes)
            try:
                item = walk.send(reply)
            except StopIteration:
                item = None

    def _fill_squareq_host(self, block_entry: BlockEntry, module: nn.Module, layout: Layout, buffer: torch.Tensor) -> None:
        """SquareQ-backed block without a GPU: the reference's host ops into the slab
        (src/stagehand/scheduler.py:290-325) — ``(f32(q) - zp) * scale`` in two fp32 roundings,
        then the cast to the runtime dtype, for each branch of the same walk."""
        for offset, nbytes, dtype, action, payload in self._squareq_actions(block_entry, module, layout, False):
            region = buffer[offset:offset + nbytes]
            if action == "dequant":
                q2d, in_flat, sv, zv = payload
                out_dim = int(q2d.shape[0])
                scale_vec = sv.to(dtype=torch.float32)[:out_dim]
                zero_vec = zv.to(dtype=torch.float32)[:out_dim]
                deq = (q2d[:, :in_flat].to(torch.float32) - zero_vec.unsqueeze(1)) * scale_vec.unsqueeze(1)
                region.view(dtype).copy_(deq.to(dtype=dtype).reshape(-1))
            elif action in ("param", "module"):
                region.view(dtype).copy_(payload.detach().to(device="cpu", dtype=dtype).reshape(-1))
            else:
                region.zero_()

    def _add_v2_file_region(self, b: SourceBuilder, path: str, spec, shape, numel: int, offset: int) -> bool:
        """A SquareQ V2 weight or bias read by the native reader: the int8 rows, scales and zero
        points are file ranges in the block source, with the branch structure of
        src/stagehand/scheduler.py:285-308. Returns False where the tensor path must run
        instead (no such layer, or a dtype that needs host work: non-int8 rows, non-fp32
        scales or zero points, fp16 biases)."""
        from stagehand_amd.squareq_v2 import read_v2_locations

        key = str(Path(path).expanduser())
        locs = self._v2_locations.get(key)
        if locs is None:
            locs = self._v2_locations[key] = read_v2_locations(key, str(Path(key).with_suffix(".manifest.json")))
        loc = locs.get(spec.layer_name)
        if loc is None:
            return False
        wf = self._weight_files.get(key, self._file_reader == "direct")
        nbytes = numel * b.runtime_dtype.itemsize
        if spec.kind == "bias":
            if "bias" not in loc:
                b.add_zero(offset, nbytes)
                return True
            off, nb, dt, _shape = loc["bias"]
            return b.add_file_param(offset, FileRange(wf, off, nb), dt, nb // dt.itemsize)
        if spec.kind != "weight" or "qweight" not in loc or "scale" not in loc:
            return False
        q_off, q_nb, q_dt, q_shape = loc["qweight"]
        s_off, s_nb, s_dt, _ = loc["scale"]
        z = loc.get("zero_point")
        if q_dt != torch.int8 or len(q_shape) == 0 or s_dt != torch.float32 or (z is not None and z[2] != torch.float32):
            return False
        out_dim = int(shape[0]) if len(shape) else 0
        in_flat = numel // max(out_dim, 1) if out_dim else 0
        if len(shape) == 0 or out_dim <= 0 or in_flat <= 0:
            b.add_zero(offset, nbytes)
            return True
        rows_q = int(q_shape[0])
        ld = q_nb // rows_q if rows_q > 0 else 0
        s_n = s_nb // 4
        z_n = z[1] // 4 if z is not None else s_n  # a missing zero point is zeros like the scales
        if min(s_n, out_dim) != out_dim or min(z_n, out_dim) != out_dim:
            b.add_zero(offset, nbytes)
            return True
        if rows_q < out_dim or ld < in_flat:
            raise ValueError(f"SquareQ layer {spec.layer_name!r}: qweight {tuple(q_shape)} is smaller than "
                             f"{out_dim}x{in_flat}")
        zp = None
        if z is not None:
            zkey = (key, spec.layer_name, out_dim)
            nonzero = self._v2_zp_nonzero.get(zkey)
            if nonzero is None:
                vals = wf.read_into(torch.empty(out_dim, dtype=torch.float32), z[0], 4 * out_dim)
                nonzero = self._v2_zp_nonzero[zkey] = bool(torch.any(vals != 0))
            zp = FileRange(wf, z[0], 4 * out_dim) if nonzero else None
        b.add_dequant_file(offset, FileRange(wf, q_off, out_dim * ld), out_dim, ld, in_flat,
                           FileRange(wf, s_off, 4 * out_dim), zp)
        return True

    # ── module-backed direct load ────────────────────────────────────

    def _load_module_backed_direct(self, block_id: str, block_entry: BlockEntry, res_entry: ResidencyEntry) -> None:
        """Module-backed block → one contiguous device buffer (src/stagehand/scheduler.py:1033-1087).

        On a GPU the bytes go through a pinned slab on the loader's copy stream
        (fp32 parameters are rounded to bf16 on the device) and the compute
        stream waits for them when the block is first used; the FSM walks
        UNLOADED → HOST_STAGED → PREFETCHING → GPU_READY at once, as in the reference.
        """
        module = block_entry.module_ref()
        if module is None:
            return
        # The parameters' host tensors written by the last save-back are pinned: the loader
        # copies them straight to the device after that copy, so the host need not wait for it.
        d2h_fence = self._d2h_fences.pop(block_id, None) if self._has_cuda else None
        if not self._has_cuda:
            self._sync_d2h_fences(block_id)
        layout = _build_param_layout(module, block_entry.dtype)
        res_entry.param_layout = layout
        numel = block_entry.size_bytes // block_entry.dtype.itemsize
        gpu_tensor = (self._engine.alloc_device(numel, block_entry.dtype) if self._has_cuda else
                      torch.empty(numel, dtype=block_entry.dtype, device=self._device))
        res_entry.gpu_tensor = gpu_tensor
        gpu_bytes = gpu_tensor.view(torch.uint8)
        if self._has_cuda:
            source = self._build_module_source(block_entry, module, layout)
            digest = self._home_load_digest(block_id, module, layout)
            res_entry.load = self._engine.submit_block_load(
                block_id, source, gpu_bytes, dest_on_loader_stream=True, wait_event=d2h_fence, pinned_pieces=True,
                digest=digest)
            if digest is None:
                self._load_digests.pop(block_id, None)
            else:
                self._load_digests[block_id] = digest
            self._unsettled.add(block_id)
            if d2h_fence is not None and any(p.grad is not None and p.grad.device.type == "cpu"
                                             for p in module.parameters()):
                # saved-back gradients move to the device on the current stream, after their save-back
                d2h_fence.wait_on(torch.cuda.current_stream().cuda_stream)
            if getattr(self._config, "frozen_host_copies", False):
                params = dict(module.named_parameters())
                keep = {}
                for name, _shape, dtype, _off, numel in layout:
                    p = params[name]
                    if (not p.requires_grad and numel > 0 and p.data.device.type == "cpu" and p.data.dtype == dtype
                            and p.data.is_contiguous()):
                        keep[name] = p.data
                if keep:
                    self._host_copies[block_id] = keep
        else:
            _flatten_params_into_buffer(module, gpu_bytes, layout)
        _restore_params_from_tensor(module, gpu_bytes, layout)
        for param in module.parameters():
            if param.grad is not None and param.grad.device.type != gpu_tensor.device.type:
                param.grad = param.grad.to(gpu_tensor.device, non_blocking=True)
        for s in (BlockState.HOST_STAGED, BlockState.PREFETCHING, BlockState.GPU_READY):
            self._residency.transition(block_id, s)
        self._telemetry.record_h2d(block_entry.size_bytes)

    def _finalize_gpu_load(self, block_id: str) -> None:
        self._residency.transition(block_id, BlockState.GPU_READY)
        block_entry = self._registry.get(block_id)
        res_entry = self._residency.get_entry(block_id)
        if res_entry.param_layout is not None and res_entry.gpu_tensor is not None:
            module = block_entry.module_ref()
            if module is not None:
                gpu_bytes = res_entry.gpu_tensor.view(torch.uint8)
                _restore_params_from_tensor(module, gpu_bytes, res_entry.param_layout)
                dev = res_entry.gpu_tensor.device
                for param in module.parameters():
                    if param.grad is not None and param.grad.device != dev:
                        param.grad = param.grad.to(dev, non_blocking=True)
        if res_entry.host_slab is not None and not hasattr(res_entry.host_slab, "pieces"):
            self._engine._pool.release(res_entry.host_slab)
        res_entry.host_slab = None

    # ── eviction ─────────────────────────────────────────────────────

    def _run_eviction(self, ignore_cooldown: bool = False) -> None:
        """Evicts by score down to the low watermark (scheduler.py:1128-1182); each eviction is
        followed by the save-back backlog bound."""
        cooldown = 0 if ignore_cooldown else self._policy.eviction_cooldown_steps
        candidates = self._residency.eviction_candidates(current_step=self._current_step, cooldown_steps=cooldown)
        protected: set[str] = set()
        base = max(self._cursor - 1, 0)
        for k in range(1, self._policy.prefetch_window + 1):
            if base + k < self._total_blocks:
                protected.add(self._ordered_blocks[base + k].block_id)
        scored: list[tuple[float, str]] = []
        for bid, _entry in candidates:
            if bid in protected:
                continue
            be = self._registry.get(bid)
            scored.append((self._policy.score_for_eviction(bid, self._cursor, be.exec_order, self._total_blocks,
                                                           be.size_bytes), bid))
        scored.sort(reverse=True)
        for _score, bid in scored:
            if self._budget.below_low_watermark():
                break
            self._evict_block(bid, save_back=not self._inference_mode, wait=False)
            self._telemetry.record_eviction()
            self._bound_save_back_backlog()

    def _bound_save_back_backlog(self) -> None:
        """Host wait for the oldest save-backs while the device memory they still hold exceeds
        the gap between the watermarks. The budget counts that memory as released (the
        reference's synchronous copy has freed it), so without a bound the memory actually
        allocated could exceed the high watermark by the whole save-back backlog."""
        wait = getattr(self._engine, "wait_releasing", None)
        if wait is None:
            return
        allowed_mb = getattr(self._config, "save_back_backlog_mb", None)
        if allowed_mb is None:
            high = getattr(self._budget, "high_watermark_mb", None)
            low = getattr(self._budget, "low_watermark_mb", None)
            if high is None or low is None:
                return
            allowed_mb = high - low
        wait(int(allowed_mb * 1024 * 1024))

    def _release_device_buffer(self, res_entry: ResidencyEntry) -> None:
        """Drop the block's device buffer; an unfinished load is waited for on the device first."""
        if res_entry.load is not None:
            self._engine.wait_device(res_entry.load)
            res_entry.load = None
        res_entry.gpu_tensor = None
        if res_entry.host_slab is not None and not hasattr(res_entry.host_slab, "pieces"):
            self._engine._pool.release(res_entry.host_slab)
        res_entry.host_slab = None

    def _evict_block(self, block_id: str, save_back: bool = False, wait: bool = True) -> None:
        """Evicts ``block_id`` (src/stagehand/scheduler.py:1184-1375). By default it returns once the
        parameters' host values are final, as the reference's synchronous eviction does; the
        eviction loop passes ``wait=False``, which leaves the save-back copies running (their
        completion is waited for before anything reads what they wrote)."""
        self._evict_block_async(block_id, save_back=save_back)
        if wait:
            self._sync_d2h_fences(block_id)

    def _evict_block_async(self, block_id: str, save_back: bool = False) -> None:
        block_entry = self._registry.get(block_id)
        res_entry = self._residency.get_entry(block_id)
        module = block_entry.module_ref()

        if block_entry.eriquant_backed:
            if self._eriquant_adapter is None:
                log.error("Block %r is eriquant-backed but no adapter set — skipping evict", block_id)
                return
            self._residency.transition(block_id, BlockState.EVICTING)
            self._eriquant_adapter.on_offload(block_id, "cpu")
            self._release_device_buffer(res_entry)
            res_entry.param_layout = None
            self._residency.transition(block_id, BlockState.UNLOADED)
            return

        module_backed = not block_entry.file_backed and not block_entry.squareq_backed
        if save_back:
            if module_backed:
                self._residency.transition(block_id, BlockState.EVICTING)
                self._await_pending_load(block_id)
                fence_before = self._d2h_fences.get(block_id)
                home = False
                if module is not None:
                    names = self._take_host_copies(block_id, module, [n for n, _ in module.named_parameters()])
                    home = self._save_block_home(block_id, module, res_entry, names)
                    if home:
                        names = []
                    self._save_params_to_host(block_id, module, names, with_grads=True)
                if home:  # the whole-block copy reads the buffer until it completes
                    self._release_with_save_back(block_id, res_entry, fence_before)
                self._release_device_buffer(res_entry)
                res_entry.param_layout = None
                self._residency.transition(block_id, BlockState.UNLOADED)
                return

            if block_entry.file_backed:
                self._residency.transition(block_id, BlockState.EVICTING)
                mutable = set(block_entry.module_param_names)
                keep_on_gpu = self._defer_backward_eviction and not self._backward_phase
                specs = {s.param_name: s for s in block_entry.file_param_specs}
                if module is not None and res_entry.param_layout is not None:
                    to_host = []
                    for name, _shape, dtype, _off, _numel in res_entry.param_layout:
                        if name in mutable:
                            if keep_on_gpu:
                                _set_param_data(module, name, _get_param_data(module, name).clone())
                            else:
                                to_host.append(name)
                        else:
                            restored = False
                            if self._backward_phase and self._defer_backward_eviction:
                                spec = specs.get(name)
                                if spec is not None:
                                    restored = self._restore_file_param_to_cpu_view(module, name, spec, dtype, block_entry)
                            if not restored:
                                _set_param_data(module, name, torch.empty(0, dtype=dtype))
                    self._save_params_to_host(block_id, module, to_host)
                    for name, param in module.named_parameters():
                        if name in mutable and param.grad is not None and param.grad.device.type != "cpu":
                            param.grad = param.grad.to("cpu", non_blocking=True)
                self._release_device_buffer(res_entry)
                res_entry.param_layout = None
                self._residency.transition(block_id, BlockState.UNLOADED)
                return

            # Generic D2H save-back through a temporary slab (src/stagehand/scheduler.py:1279-1331).
            self._residency.transition(block_id, BlockState.EVICTING)
            if res_entry.gpu_tensor is not None:
                self._await_pending_load(block_id)
                slab = self._engine._pool.acquire(block_entry.size_bytes)
                handle = self._engine.submit_d2h(block_id, res_entry.gpu_tensor, slab)
                self._engine.wait(handle)
                self._telemetry.record_d2h(res_entry.gpu_tensor.numel() * res_entry.gpu_tensor.element_size())
                if module is not None and res_entry.param_layout is not None:
                    _restore_params_from_tensor(module, slab.buffer, res_entry.param_layout)
                    for name, *_rest in res_entry.param_layout:
                        _set_param_data(module, name, _get_param_data(module, name).clone())
                self._engine._pool.release(slab)
                res_entry.host_slab = None
            if module is not None:
                for param in module.parameters():
                    if param.grad is not None and param.grad.device.type != "cpu":
                        param.grad = param.grad.to("cpu", non_blocking=True)
            self._release_device_buffer(res_entry)
            self._residency.transition(block_id, BlockState.UNLOADED)
            return

        # No save-back: GPU_READY → GPU_FREEING → UNLOADED.
        self._residency.transition(block_id, BlockState.GPU_FREEING)
        if module is not None and res_entry.param_layout is not None:
            if module_backed:
                self._await_pending_load(block_id)
                names = self._take_host_copies(block_id, module, [n for n, *_ in res_entry.param_layout])
                self._save_params_to_host(block_id, module, names)
            elif block_entry.file_backed:  # SquareQ-backed blocks are file-backed too (registry BlockEntry.file_backed)
                resident = set(block_entry.module_param_names)
                keep_on_gpu = self._defer_backward_eviction and not self._backward_phase
                to_host = []
                for name, _shape, dtype, _off, _numel in res_entry.param_layout:
                    if name in resident:
                        if keep_on_gpu:
                            _set_param_data(module, name, _get_param_data(module, name).clone())
                        else:
                            to_host.append(name)
                    else:
                        _set_param_data(module, name, torch.empty(0, dtype=dtype))
                self._save_params_to_host(block_id, module, to_host)
            else:
                _detach_params(module, res_entry.param_layout)
        self._release_device_buffer(res_entry)
        res_entry.param_layout = None
        self._residency.transition(block_id, BlockState.UNLOADED)

    def _restore_file_param_to_cpu_view(self, module: nn.Module, name: str, spec: FileParamSpec, runtime_dtype: torch.dtype,
                                        block_entry: BlockEntry) -> bool:
        sharded = block_entry.source_format == "safetensors_sharded"
        path = spec.file_path if (spec.file_path and sharded) else str(block_entry.source_path)
        t = self._get_file_tensor_view(path, spec)
        if spec.source_dtype != runtime_dtype:
            t = t.to(dtype=runtime_dtype)
        _set_param_data(module, name, t)
        return True
