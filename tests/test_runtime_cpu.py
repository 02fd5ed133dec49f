"""CPU tests of StagehandRuntime block mode around training with activation
checkpointing (host path; the device path is covered by the GPU tests).

Non-reentrant checkpointing re-runs a block's forward inside the backward pass
and may stop that forward early, so the block's forward post-hook does not
always run; the runtime must still end every step with all references
released, so that blocks stay evictable (the reference's hooks,
src/stagehand/__init__.py:452-548, leak a reference per block here).
"""
from __future__ import annotations

import pytest
import torch

import stagehand_amd as stagehand
from stagehand_amd.residency import BlockState
from bench_workloads import TRAIN_BLOCK_PATTERN, TrainDiT, init_train_dit_

pytestmark = pytest.mark.skipif(torch.cuda.is_available(), reason="host-path runtime tests (no GPU)")


def _resident(rt) -> int:
    return sum(1 for e in rt.registry.blocks_in_order() if rt.residency.get_state(e.block_id) == BlockState.GPU_READY)


@pytest.mark.parametrize("checkpoint", [True, False])
def test_checkpointed_training_releases_every_reference(checkpoint):
    model = init_train_dit_(TrainDiT(depth=6, hidden=64, heads=4, mlp_ratio=2.0, rank=4, checkpoint=checkpoint), 0)
    ref = init_train_dit_(TrainDiT(depth=6, hidden=64, heads=4, mlp_ratio=2.0, rank=4, checkpoint=checkpoint), 0)
    cfg = stagehand.StagehandConfig(pinned_pool_mb=64, pinned_slab_mb=4, vram_high_watermark_mb=2,
                                    vram_low_watermark_mb=1, prefetch_window_blocks=3, nan_inf_check=False,
                                    strict_bf16=False, telemetry_enabled=True)
    cfg.telemetry_file = None
    rt = stagehand.StagehandRuntime(model, cfg, block_pattern=TRAIN_BLOCK_PATTERN, dtype=torch.bfloat16,
                                    inference_mode=False)
    # a budget that counts resident blocks: above the high watermark with more than 2
    rt._budget.above_high_watermark = lambda: _resident(rt) > 2
    rt._budget.below_low_watermark = lambda: _resident(rt) <= 1
    rt._budget.can_prefetch = lambda: _resident(rt) <= 2
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1, 8, 64, generator=g).bfloat16()
    ctx = torch.randn(1, 4, 64, generator=g).bfloat16()
    vec = torch.randn(1, 64, generator=g).bfloat16()
    for step in range(3):
        xi = x.clone().requires_grad_()
        rt.begin_step(step)
        with rt.managed_forward(), rt.managed_backward():
            y = model(xi, ctx, vec)
            y.float().square().mean().backward()
        rt.end_step()
        assert [rt.residency.get_entry(e.block_id).refcount for e in rt.registry.blocks_in_order()] == [0] * 6
        assert rt.telemetry.history[-1].evictions > 0
        assert _resident(rt) <= 3
    xr = x.clone().requires_grad_()
    yr = ref(xr, ctx, vec)
    yr.float().square().mean().backward()
    assert torch.equal(y, yr)
    for (n, p), (_m, q) in zip(model.named_parameters(), ref.named_parameters()):
        if "lora" in n:
            # three accumulated backward passes against one
            assert torch.allclose(p.grad.float(), 3 * q.grad.float(), rtol=2e-2, atol=1e-4), n
    rt.shutdown()


def test_hardware_queue_hint_logs_once_below_eight(monkeypatch, caplog):
    """Training with changed-chunk save-backs logs one hint when HIP has fewer than 8 hardware
    queues, and none with 8."""
    import logging

    from stagehand_amd import runtime as rt_mod

    for queues, expect in (("4", 1), ("8", 0)):
        monkeypatch.setattr(rt_mod, "_HW_QUEUES_HINTED", False)
        monkeypatch.setenv("GPU_MAX_HW_QUEUES", queues)
        caplog.clear()
        with caplog.at_level(logging.INFO, logger="stagehand_amd.runtime"):
            rt_mod._hint_hw_queues()
            rt_mod._hint_hw_queues()
        assert sum("hardware queues" in r.getMessage() for r in caplog.records) == expect, queues
