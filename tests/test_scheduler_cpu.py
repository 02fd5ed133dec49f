"""CPU tests of the block scheduler (hooks' target) with mock pool and budget.

Restates the scenarios of the reference's tests/test_scheduler.py:225-609
(lifecycle, prefetch, stall accounting, eviction with refcount and
prefetch-window protection, inference save-back rule, guards) against
``stagehand_amd.scheduler.StagehandScheduler``. Without a GPU the scheduler
takes the reference's host path (module params flattened into a CPU buffer),
so these pin control flow, FSM walks and telemetry counts, not kernels.
"""
from __future__ import annotations

from unittest.mock import MagicMock

import pytest
import torch
from torch import nn

from stagehand_amd.config import StagehandConfig
from stagehand_amd.registry import BlockRegistry
from stagehand_amd.residency import BlockState, ResidencyMap
from stagehand_amd.scheduler import StagehandScheduler, StaticLookaheadPolicy
from stagehand_amd.telemetry import StagehandTelemetry
from stagehand_amd.transfer import AsyncTransferEngine

pytestmark = pytest.mark.skipif(torch.cuda.is_available(), reason="host-path scheduler tests (no GPU)")


class Budget:
    def __init__(self, above: bool = False, prefetch: bool = True) -> None:
        self.above, self.below, self.prefetch = above, True, prefetch

    def above_high_watermark(self) -> bool:
        return self.above

    def below_low_watermark(self) -> bool:
        return self.below

    def can_prefetch(self) -> bool:
        return self.prefetch


class Guards:
    def __init__(self, nan: int = 0, inf: int = 0) -> None:
        self.nan, self.inf, self.seen = nan, inf, []

    def check_output(self, tensor, block_id, step):
        self.seen.append(block_id)
        return self.nan, self.inf


class Slab:
    def __init__(self, n: int) -> None:
        self.slab_id, self.pool_id, self.size_bytes = 0, 0, n
        self.buffer = torch.zeros(n, dtype=torch.uint8)


class Pool:
    slab_bytes = 256 * 1024
    num_slabs = 8

    def __init__(self) -> None:
        self.acquired = self.released = 0

    def acquire(self, size_bytes: int) -> Slab:
        self.acquired += 1
        return Slab(size_bytes)

    def release(self, slab) -> None:
        self.released += 1


def _stack(n: int = 10, window: int = 3, above: bool = False, guards=None, inference: bool = False, model=None):
    if model is None:
        model = nn.Sequential()
        for i in range(n):
            model.add_module(f"block_{i}", nn.Linear(16, 16, bias=False))
    reg = BlockRegistry()
    reg.build_from_model(model, block_pattern=r"block_\d+", group="test", dtype=torch.bfloat16)
    reg.validate(pool_capacity_bytes=10 << 20)
    res = ResidencyMap(reg)
    pool = Pool()
    budget = Budget(above=above)
    tel = StagehandTelemetry(enabled=True, interval_steps=100)
    sched = StagehandScheduler(registry=reg, residency=res, transfer_engine=AsyncTransferEngine(pool=pool, max_inflight=4),
                               budget=budget, policy=StaticLookaheadPolicy(prefetch_window=window, eviction_cooldown_steps=2),
                               guards=guards, telemetry=tel, config=StagehandConfig(), inference_mode=inference)
    return sched, budget, tel, res, reg, pool, model


def _run_step(sched, reg, step, output=None):
    sched.begin_step(step)
    for e in reg.blocks_in_order():
        sched.before_block(e.block_id)
        sched.after_block(e.block_id, output)
    sched.end_step()


def test_steps_record_history_and_restore_weights():
    sched, _b, tel, res, reg, _p, model = _stack(n=5, window=2)
    want = [m.weight.detach().to(torch.bfloat16).clone() for m in model]
    for step in range(3):
        _run_step(sched, reg, step, torch.randn(16))
    assert [m.step for m in tel._history] == [0, 1, 2]
    for m, w in zip(model, want):
        assert m.weight.dtype == torch.bfloat16 and torch.equal(m.weight, w)
    assert all(res.get_state(e.block_id) == BlockState.GPU_READY for e in reg.blocks_in_order())


def test_prefetch_reaches_lookahead_blocks():
    sched, _b, _t, res, reg, _p, _m = _stack(n=10, window=3)
    order = reg.blocks_in_order()
    sched.begin_step(0)
    sched.before_block(order[0].block_id)
    sched.after_block(order[0].block_id)
    # blocks 1..3 left UNLOADED by the prefetch
    assert all(res.get_state(order[i].block_id) != BlockState.UNLOADED for i in (1, 2, 3))
    assert res.get_state(order[4].block_id) == BlockState.UNLOADED
    sched.end_step()


def test_cold_blocks_count_as_misses_and_warm_as_hits():
    sched, _b, tel, _r, reg, _p, _m = _stack(n=3, window=0)
    sched.begin_step(0)
    first = reg.blocks_in_order()[0].block_id
    sched.before_block(first)
    sched.after_block(first)
    assert tel._current is not None and tel._current.prefetch_misses >= 1
    sched.end_step()

    sched2, _b, tel2, _r, reg2, _p, _m = _stack(n=3, window=0)
    _run_step(sched2, reg2, 0)
    assert tel2._history[0].prefetch_misses == 3
    _run_step(sched2, reg2, 1)  # nothing evicted: every block is resident
    assert tel2._history[1].prefetch_hits == 3 and tel2._history[1].prefetch_misses == 0


def test_referenced_block_is_never_evictable():
    sched, budget, _t, res, reg, _p, _m = _stack(n=3, window=0, above=True)
    budget.below = False
    first = reg.blocks_in_order()[0].block_id
    sched.begin_step(0)
    sched.before_block(first)
    assert res.get_entry(first).refcount > 0 and not res.can_evict(first)
    sched.after_block(first)
    sched.end_step()


def test_eviction_above_watermark_frees_blocks():
    sched, budget, tel, res, reg, _p, _m = _stack(n=5, window=1, above=False)
    _run_step(sched, reg, 0)
    budget.above, budget.below = True, False
    sched.begin_step(5)
    first = reg.blocks_in_order()[0].block_id
    sched.before_block(first)
    sched.after_block(first)
    sched.end_step()
    evicted = sum(m.evictions for m in tel._history)
    assert evicted >= 1
    assert any(res.get_state(e.block_id) != BlockState.GPU_READY for e in reg.blocks_in_order())


def test_prefetch_window_is_protected_from_eviction():
    sched, budget, _t, res, reg, _p, _m = _stack(n=10, window=3, above=True)
    budget.below = False
    _run_step(sched, reg, 0)
    order = reg.blocks_in_order()
    sched.begin_step(10)
    for i in range(3):
        sched.before_block(order[i].block_id)
        sched.after_block(order[i].block_id)
    for i in (3, 4, 5):
        assert res.get_state(order[i].block_id) in (BlockState.GPU_READY, BlockState.PREFETCHING, BlockState.HOST_STAGED)
    sched.end_step()


@pytest.mark.parametrize("inference,want", [(True, False), (False, True)])
def test_save_back_rule(inference, want):
    """``save_back = not inference_mode`` for every block kind (scheduler.py:1179-1181); a
    module-backed block's data still survives an inference eviction (scheduler.py:1340-1352)."""
    for file_backed in (False, True):
        sched, budget, *_ = _stack(n=1, window=0, above=True, inference=inference)
        budget.below = False
        fake = MagicMock(exec_order=0, size_bytes=1024, file_backed=file_backed, squareq_backed=False)
        sched._registry.get = MagicMock(return_value=fake)
        sched._residency.eviction_candidates = MagicMock(return_value=[("block_0", MagicMock())])
        sched._policy.score_for_eviction = MagicMock(return_value=1.0)
        sched._budget.below_low_watermark = MagicMock(side_effect=[False, True])
        sched._evict_block = MagicMock()  # the reference's interception point (tests/test_scheduler.py:495-528)
        sched._run_eviction()
        assert sched._evict_block.call_count == 1
        _args, kwargs = sched._evict_block.call_args
        assert kwargs["save_back"] is want
        assert kwargs["wait"] is False  # the loop leaves save-backs running


def test_inference_eviction_keeps_module_backed_values():
    sched, budget, _t, res, reg, _p, model = _stack(n=4, window=0, inference=True)
    want = [m.weight.detach().to(torch.bfloat16).clone() for m in model]
    _run_step(sched, reg, 0)
    budget.above, budget.below = True, False
    sched._run_eviction(ignore_cooldown=True)
    assert all(res.get_state(e.block_id) != BlockState.GPU_READY for e in reg.blocks_in_order())
    budget.above, budget.below = False, True
    _run_step(sched, reg, 1)
    for m, w in zip(model, want):
        assert torch.equal(m.weight, w)


def test_guards_see_outputs_only():
    g = Guards(nan=2, inf=1)
    sched, _b, tel, _r, reg, _p, _m = _stack(n=3, guards=g)
    _run_step(sched, reg, 0, torch.randn(4))
    assert len(g.seen) == 3
    assert (tel._history[0].nan_count, tel._history[0].inf_count) == (6, 3)
    g2 = Guards()
    sched2, _b, _t, _r, reg2, _p, _m = _stack(n=2, guards=g2)
    _run_step(sched2, reg2, 0, None)
    assert g2.seen == []


def test_direct_eviction_waits_for_its_save_back_but_the_loop_does_not():
    """``_evict_block`` returns with the block's host values final, as the reference's synchronous
    eviction does (scheduler.py:1184-1375); the eviction loop leaves save-backs running."""
    sched, budget, *_ = _stack(n=2, window=0, above=True)
    calls = []
    sched._evict_block_async = MagicMock(side_effect=lambda bid, save_back=False: calls.append(("evict", bid)))
    sched._sync_d2h_fences = MagicMock(side_effect=lambda bid=None: calls.append(("sync", bid)))
    sched._evict_block("block_0", save_back=True)
    assert calls == [("evict", "block_0"), ("sync", "block_0")]
    calls.clear()
    fake = MagicMock(exec_order=0, size_bytes=1024, file_backed=False, squareq_backed=False)
    sched._registry.get = MagicMock(return_value=fake)
    sched._residency.eviction_candidates = MagicMock(return_value=[("block_1", MagicMock())])
    sched._policy.score_for_eviction = MagicMock(return_value=1.0)
    sched._budget.below_low_watermark = MagicMock(side_effect=[False, True])
    sched._run_eviction()
    assert calls == [("evict", "block_1")]


def test_save_back_fence_follows_the_last_use_and_the_step_start():
    """Which events a module-backed block's save-back waits for (host logic; the events are
    recorded on the device in real runs, stand-ins here): outside a step and in inference, the whole
    queue (None); inside a step, the step's start and the block's last use (its after_block or a
    gradient accumulation into it); the whole queue again once a parameter changed in place or the
    block was loaded after its last hook. The gradient hooks last from begin_step to end_step."""
    events = []

    def record():
        events.append(object())
        return events[-1]

    def begin(sched, step):
        # begin_step with the device-only bookkeeping switched on
        sched._has_cuda = True
        try:
            sched.begin_step(step)
        finally:
            sched._has_cuda = False

    sched, _b, _t, _res, reg, _p, model = _stack(n=3, window=1)
    sched._engine.record_event = record
    assert sched._save_back_fence("block_1", model.block_1) is None
    begin(sched, 0)
    step_mark = events[-1]
    assert len(sched._grad_hooks) == 3  # one per trainable parameter of the three blocks
    assert sched._save_back_fence("block_1", model.block_1) == [step_mark]
    sched.before_block("block_1")
    sched.after_block("block_1")
    assert sched._save_back_fence("block_1", model.block_1) == [events[-1], step_mark]
    # a gradient accumulated into block 0 marks its last use
    model.block_0(torch.randn(2, 16, dtype=model.block_0.weight.dtype)).float().sum().backward()
    assert sched._save_back_fence("block_0", model.block_0) == [events[-1], step_mark]
    # a block loaded again since its last hook: the whole queue, until its next after_block
    sched._unsettled.add("block_2")
    assert sched._save_back_fence("block_2", model.block_2) is None
    sched.before_block("block_2")
    sched.after_block("block_2")
    assert sched._save_back_fence("block_2", model.block_2) == [events[-1], step_mark]
    # a parameter changed in place since the step began: the whole queue
    with torch.no_grad():
        model.block_1.weight.add_(1.0)
    assert sched._save_back_fence("block_1", model.block_1) is None
    sched.end_step()
    assert sched._grad_hooks == [] and sched._save_back_fence("block_2", model.block_2) is None

    inf, *_rest, inf_model = _stack(n=2, window=1, inference=True)
    inf._engine.record_event = record
    begin(inf, 0)
    assert inf._save_back_fence("block_0", inf_model.block_0) is None and inf._grad_hooks == []
