"""CPU tests of the control plane the data path drives: registry, residency
FSM, budget watermarks, numeric guards, lookahead policy.

Each class restates the behaviour pinned by the reference's own tests
(tests/test_registry.py:60-609, tests/test_scheduler.py:143-221) against this
package's modules, which keep the reference's names and semantics.
"""
from __future__ import annotations

from unittest import mock

import pytest
import torch
from torch import nn

from stagehand_amd.budget import BudgetManager
from stagehand_amd.errors import DtypeMismatchError, InvalidStateTransitionError, StagehandOOMError
from stagehand_amd.guards import NumericGuard
from stagehand_amd.registry import BlockRegistry
from stagehand_amd.residency import VALID_TRANSITIONS, BlockState, ResidencyMap
from stagehand_amd.scheduler import StaticLookaheadPolicy

S = BlockState


def _model(n: int, fin: int = 64, fout: int = 64) -> nn.Module:
    m = nn.Module()
    m.add_module("block", nn.ModuleList(nn.Linear(fin, fout) for _ in range(n)))
    return m


def _registry(n: int = 4, dtype: torch.dtype = torch.bfloat16, fin: int = 64) -> BlockRegistry:
    reg = BlockRegistry()
    reg.build_from_model(_model(n, fin, fin), block_pattern=r"^block\.\d+$", group="wan", dtype=dtype)
    reg.validate(pool_capacity_bytes=1 << 30)
    return reg


def _to_gpu_ready(rmap: ResidencyMap, bid: str) -> None:
    for s in (S.HOST_STAGED, S.PREFETCHING, S.GPU_READY):
        rmap.transition(bid, s)


# ── registry (reference tests/test_registry.py:60-265) ──────────────────


class TestRegistry:
    def test_count_order_groups_membership(self):
        reg = _registry(6)
        assert len(reg) == 6
        assert [e.exec_order for e in reg.blocks_in_order()] == list(range(6))
        assert [e.block_id for e in reg.blocks_in_order()] == [f"block.{i}" for i in range(6)]
        assert len(reg.groups()["wan"]) == 6
        assert "block.0" in reg and "block.5" in reg and "block.6" not in reg
        assert reg.get("block.2").group == "wan"
        with pytest.raises(KeyError):
            reg.get("missing")

    def test_size_bytes_uses_the_passed_dtype(self):
        # registry.py:69-74 sums numel * dtype.itemsize of the dtype passed in
        # (the reference's test_size_bytes_calculation expects fp32 bytes and
        # fails against its own code; the code is what is restated here).
        for dtype in (torch.bfloat16, torch.float16, torch.float32):
            reg = BlockRegistry()
            reg.build_from_model(_model(1, 1024, 1024), r"^block\.\d+$", "wan", dtype)
            e = reg.blocks_in_order()[0]
            assert e.size_bytes == (1024 * 1024 + 1024) * dtype.itemsize
            assert e.dtype == dtype

    def test_validate_oversized_and_freeze(self):
        reg = BlockRegistry()
        reg.build_from_model(_model(1), r"^block\.\d+$", "wan", torch.bfloat16)
        with pytest.raises(StagehandOOMError, match="exceeds pool capacity"):
            reg.validate(pool_capacity_bytes=1)
        reg2 = _registry(2)
        with pytest.raises(RuntimeError, match="frozen"):
            reg2.build_from_model(_model(1), r"^block\.\d+$", "dit", torch.bfloat16)

    def test_module_ref_is_weak(self):
        model = _model(1)
        reg = BlockRegistry()
        reg.build_from_model(model, r"^block\.\d+$", "wan", torch.bfloat16)
        e = reg.blocks_in_order()[0]
        assert e.module_ref() is model.block[0]

    def test_squareq_v1_conversion(self, tmp_path):
        """A v1 slab converts weight + bias of a frozen Linear and drops the module tensors
        (reference tests/test_registry.py:202-251)."""
        path = tmp_path / "tiny.fpk"
        torch.save({"manifest": {"model_name": "tiny", "layout": "rowwise_sym_int8", "pack_k": 1,
                                 "layers": [{"name": "block.0", "out": 8, "inp": 8, "padded_in": 8, "has_bias": True}]},
                    "layers": {"block.0": {"qweight": torch.randint(-127, 128, (8, 8), dtype=torch.int8),
                                           "scale": torch.ones(8), "zero_point": torch.zeros(8), "bias": torch.zeros(8)}}},
                   path)
        model = _model(1, 8, 8)
        model.requires_grad_(False)
        reg = BlockRegistry()
        reg.build_from_model(model, r"^block\.\d+$", "wan", torch.float32)
        reg.validate(pool_capacity_bytes=1 << 30)
        assert reg.convert_to_file_backed(str(path)) == 2
        e = reg.get("block.0")
        assert e.file_backed and e.squareq_backed and e.source_format == "squareq_bp8"
        assert len(e.squareq_param_specs) == 2
        blk = e.module_ref()
        assert blk.weight.numel() == 0 and blk.bias.numel() == 0

    def test_trainable_params_stay_module_backed(self, tmp_path):
        """Params with requires_grad keep their module tensors (registry.py:505-510)."""
        from safetensors.torch import save_file

        model = _model(2, 8, 8)
        path = tmp_path / "w.safetensors"
        save_file({k: v.detach().clone() for k, v in model.state_dict().items()}, str(path))
        model.block[0].requires_grad_(False)  # block 1 stays trainable
        reg = BlockRegistry()
        reg.build_from_model(model, r"^block\.\d+$", "wan", torch.float32)
        reg.validate(pool_capacity_bytes=1 << 30)
        assert reg.convert_to_file_backed(str(path)) == 2
        assert reg.get("block.0").file_backed and not reg.get("block.1").file_backed
        assert model.block[0].weight.numel() == 0 and model.block[1].weight.numel() == 64

    def test_wan_key_aliases(self):
        """reference tests/test_registry.py:253-265."""
        keys = BlockRegistry._candidate_tensor_keys
        assert "blocks.0.self_attn.q.weight" in keys("blocks.0", "attn1.to_q.orig.weight")
        assert "blocks.0.cross_attn.o.bias" in keys("blocks.0", "attn2.to_out.0.orig.bias")
        assert "blocks.0.ffn.0.weight" in keys("blocks.0", "ffn.net.0.proj.orig.weight")
        assert "blocks.0.modulation" in keys("blocks.0", "scale_shift_table")


# ── residency FSM (reference tests/test_registry.py:271-420) ───────────


class TestResidency:
    def test_legal_paths(self):
        reg = _registry(1)
        for tail in ([S.GPU_FREEING, S.UNLOADED], [S.EVICTING, S.HOST_STAGED], [S.EVICTING, S.UNLOADED]):
            rmap = ResidencyMap(reg)
            for s in [S.HOST_STAGED, S.PREFETCHING, S.GPU_READY] + tail:
                rmap.transition("block.0", s)
                assert rmap.get_state("block.0") == s

    def test_every_illegal_transition_raises(self):
        reg = _registry(1)
        illegal = 0
        for src in S:
            for dst in S:
                if dst in VALID_TRANSITIONS.get(src, frozenset()):
                    continue
                rmap = ResidencyMap(reg)
                rmap.get_entry("block.0").state = src
                with pytest.raises(InvalidStateTransitionError):
                    rmap.transition("block.0", dst)
                illegal += 1
        assert illegal == 36 - 8  # six states, eight legal edges (residency.py:45-52)

    def test_refcount_and_candidates(self):
        reg = _registry(3)
        rmap = ResidencyMap(reg)
        assert all(rmap.get_entry(f"block.{i}").state == S.UNLOADED for i in range(3))
        with pytest.raises(ValueError):
            rmap.decrement_ref("block.0")
        for i, last in enumerate((5, 8, 10)):
            _to_gpu_ready(rmap, f"block.{i}")
            rmap.get_entry(f"block.{i}").last_used_step = last
        assert sorted(rmap.gpu_resident_blocks()) == ["block.0", "block.1", "block.2"]
        assert rmap.can_evict("block.0")
        rmap.increment_ref("block.0")
        assert not rmap.can_evict("block.0")
        assert sorted(b for b, _ in rmap.eviction_candidates(current_step=10, cooldown_steps=2)) == ["block.1"]
        rmap.decrement_ref("block.0")
        assert sorted(b for b, _ in rmap.eviction_candidates(current_step=10, cooldown_steps=2)) == ["block.0", "block.1"]
        assert len(rmap) == 3 and "block.1" in rmap and "nope" not in rmap


# ── budget (reference tests/test_registry.py:426-489) ───────────────────


class TestBudget:
    def test_invalid_watermarks(self):
        for hi, lo in ((1000, 2000), (1000, 1000)):
            with pytest.raises(ValueError, match="must be greater"):
                BudgetManager(high_watermark_mb=hi, low_watermark_mb=lo)

    @pytest.mark.parametrize("used_mb,above,below,prefetch", [(120, True, False, False), (30, False, True, True),
                                                               (75, False, False, True)])
    def test_predicates(self, used_mb, above, below, prefetch):
        bm = BudgetManager(high_watermark_mb=100, low_watermark_mb=50)
        with mock.patch("torch.cuda.is_available", return_value=True), \
                mock.patch("torch.cuda.memory_allocated", return_value=used_mb << 20):
            assert bm.above_high_watermark() is above
            assert bm.should_evict() is above
            assert bm.below_low_watermark() is below
            assert bm.can_prefetch() is prefetch
            assert bm.headroom_mb() == pytest.approx(100 - used_mb)

    def test_memory_held_by_save_backs_counts_as_released(self):
        """Device memory an eviction gave up, still held by its asynchronous save-back, is left out
        (the reference's synchronous copy has freed it when the eviction loop checks again)."""
        bm = BudgetManager(high_watermark_mb=100, low_watermark_mb=50)
        releasing = [0]
        bm.count_as_released(lambda: releasing[0])
        with mock.patch("torch.cuda.is_available", return_value=True), \
                mock.patch("torch.cuda.memory_allocated", return_value=120 << 20):
            assert bm.above_high_watermark() and not bm.below_low_watermark()
            releasing[0] = 80 << 20
            assert bm.vram_used_mb() == pytest.approx(40.0)
            assert bm.below_low_watermark() and not bm.above_high_watermark()
            releasing[0] = 500 << 20  # never below zero
            assert bm.vram_used_mb() == 0.0
        bm.count_as_released(None)
        with mock.patch("torch.cuda.is_available", return_value=True), \
                mock.patch("torch.cuda.memory_allocated", return_value=120 << 20):
            assert bm.vram_used_mb() == pytest.approx(120.0)

    def test_without_gpu(self):
        bm = BudgetManager(high_watermark_mb=100, low_watermark_mb=50)
        with mock.patch("torch.cuda.is_available", return_value=False):
            assert bm.vram_used_mb() == 0.0 and bm.vram_reserved_mb() == 0.0
            assert bm.can_prefetch() and not bm.should_evict()
        with mock.patch("torch.cuda.is_available", return_value=True), \
                mock.patch("torch.cuda.memory_reserved", return_value=200 << 20):
            assert bm.vram_reserved_mb() == pytest.approx(200.0)


# ── guards (reference tests/test_registry.py:495-609) ───────────────────


class TestGuards:
    def test_dtype(self):
        NumericGuard(strict_bf16=True).check_dtype(torch.zeros(2, dtype=torch.bfloat16), torch.bfloat16, "b")
        with pytest.raises(DtypeMismatchError, match="expected.*bfloat16.*got.*float32"):
            NumericGuard(strict_bf16=True).check_dtype(torch.zeros(2), torch.bfloat16, "b")
        NumericGuard(strict_bf16=False).check_dtype(torch.zeros(2), torch.bfloat16, "b")

    @pytest.mark.parametrize("vals,nan,inf", [([1.0, float("nan"), 3.0], 1, 0),
                                              ([1.0, float("inf"), float("-inf"), 4.0], 0, 2),
                                              ([float("nan"), float("inf"), float("nan"), 1.0], 2, 1),
                                              ([0.5] * 100, 0, 0)])
    def test_output_counts(self, vals, nan, inf):
        assert NumericGuard(nan_inf_check=True).check_output(torch.tensor(vals), "b", 0) == (nan, inf)
        assert NumericGuard(nan_inf_check=False).check_output(torch.tensor(vals), "b", 0) == (0, 0)

    def test_promotion(self):
        g = NumericGuard(fail_on_dtype_promotion=True)
        for a, b in ((torch.bfloat16, torch.float32), (torch.float16, torch.float32)):
            with pytest.raises(DtypeMismatchError, match="promotion"):
                g.check_promotion(a, b, "c")
        for a, b in ((torch.bfloat16, torch.bfloat16), (torch.float32, torch.bfloat16), (torch.bfloat16, torch.float16),
                     (torch.int8, torch.float32)):
            g.check_promotion(a, b, "c")
        NumericGuard(fail_on_dtype_promotion=False).check_promotion(torch.bfloat16, torch.float32, "c")


# ── lookahead policy (reference tests/test_scheduler.py:143-221) ────────


class TestPolicy:
    @pytest.mark.parametrize("window,cursor,total,want", [(3, 2, 10, [3, 4, 5]), (3, 8, 10, [9]), (3, 9, 10, []),
                                                          (1, 0, 5, [1]), (0, 0, 5, [])])
    def test_window(self, window, cursor, total, want):
        assert StaticLookaheadPolicy(prefetch_window=window).blocks_to_prefetch(cursor, total, {}) == want

    @pytest.mark.parametrize("order,cursor,size,want", [(7, 2, 1000, 5000), (1, 8, 500, 1500), (5, 5, 200, 2000)])
    def test_eviction_score(self, order, cursor, size, want):
        # distance to next use (exec_order - cursor) mod n, a block at the cursor counting n
        p = StaticLookaheadPolicy()
        assert p.score_for_eviction(block_id="b", current_cursor=cursor, entry_exec_order=order, total_blocks=10,
                                    size_bytes=size) == want

    def test_cooldown(self):
        p = StaticLookaheadPolicy(eviction_cooldown_steps=2)
        assert [p.should_evict(5, s) for s in (6, 7, 8)] == [False, False, True]
        p0 = StaticLookaheadPolicy(eviction_cooldown_steps=0)
        assert [p0.should_evict(5, s) for s in (5, 6)] == [False, True]
