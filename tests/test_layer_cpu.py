"""CPU tests of layer mode (``stagehand_amd.layer`` / ``LayerRuntime``).

Restates the reference's tests/test_layer.py:128-583 (discovery, budget
parsing, auto pool sizing, trace → rebuild → auto-step, backward, shutdown,
the top-level API) and runs BASELINE config 1 — the reference's CPU plumbing
case — end to end: 8 × Linear(4096, 4096) fp32, bf16 storage, prefetch_k=3,
inference mode, a trace step then a scheduled step, checking the outputs and
every packed byte against the closed-form bf16 rounding (oracle).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

import stagehand_amd as stagehand
from stagehand_amd.layer import LayerRuntime, _auto_pool_config, _discover_layers, _next_power_of_two, _parse_budget

pytestmark = pytest.mark.skipif(torch.cuda.is_available(), reason="host-path layer tests (no GPU)")


class Seq(nn.Module):
    def __init__(self, n: int = 5, hidden: int = 32) -> None:
        super().__init__()
        self.layers = nn.ModuleList(nn.Linear(hidden, hidden, bias=False) for _ in range(n))

    def forward(self, x):
        for layer in self.layers:
            x = layer(x)
        return x


class Mixed(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.embed = nn.Embedding(100, 32)
        self.conv = nn.Conv2d(1, 8, 3, padding=1)
        self.fc = nn.Linear(32, 16)


class Shared(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.a = nn.Linear(32, 32, bias=False)
        self.b = self.a
        self.c = nn.Linear(32, 32, bias=False)

    def forward(self, x):
        return self.c(self.b(self.a(x)))


class Reversed(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.a, self.b, self.c = (nn.Linear(32, 32, bias=False) for _ in range(3))

    def forward(self, x):
        return self.a(self.b(self.c(x)))


class Nested(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.block = nn.Sequential(nn.Linear(32, 32), nn.Sequential(nn.Linear(32, 32), nn.Linear(32, 16)))
        self.head = nn.Linear(16, 4)


# ── discovery, budgets, auto-config (reference tests/test_layer.py:146-245) ──


def test_discovery():
    assert len(_discover_layers(Seq(5))) == 5
    assert {type(m) for _, m in _discover_layers(Mixed())} == {nn.Linear, nn.Conv2d, nn.Embedding}
    assert len(_discover_layers(Mixed(), target_types=(nn.Linear,))) == 1
    assert len(_discover_layers(Shared())) == 2
    assert len(_discover_layers(Nested())) == 4
    assert _discover_layers(nn.Sequential(nn.BatchNorm1d(4))) == []


@pytest.mark.parametrize("value,want", [(None, None), (4 << 30, 4 << 30), ("4GB", 4 << 30), ("512MB", 512 << 20),
                                        ("2gb", 2 << 30), ("1048576", 1048576)])
def test_parse_budget(value, want):
    assert _parse_budget(value) == want


def test_auto_pool_config():
    layers = _discover_layers(Seq(3, 32))
    cfg = _auto_pool_config(layers, torch.bfloat16, prefetch_k=3, vram_budget=None, ram_budget=None)
    assert cfg.pinned_slab_mb & (cfg.pinned_slab_mb - 1) == 0
    assert cfg.pinned_pool_mb // cfg.pinned_slab_mb >= 7
    cfg8 = _auto_pool_config(layers, torch.bfloat16, prefetch_k=3, vram_budget=8 << 30, ram_budget=None)
    assert cfg8.vram_low_watermark_mb < cfg8.vram_high_watermark_mb < 8192
    assert [_next_power_of_two(n) for n in (0, 1, 3, 4, 5)] == [1, 1, 4, 4, 8]


# ── trace → rebuild → scheduled (reference tests/test_layer.py:251-346) ──


def test_trace_rebuild_autostep():
    model = Seq(4)
    rt = LayerRuntime(model, dtype=torch.float32, prefetch_k=2, telemetry=False)
    assert (rt.mode, rt.traced, rt.step, rt.num_layers) == ("trace", False, 0, 4)
    assert isinstance(rt.stats, dict)
    x = torch.randn(2, 32)
    y0 = model(x)
    assert rt.mode == "trace" and rt.step == 0 and len(rt.trace_order) == 4
    y1 = model(x)
    assert (rt.mode, rt.traced, rt.step) == ("scheduled", True, 1)
    for want in (2, 3):
        model(x)
        assert rt.step == want
    assert torch.equal(y0, y1)
    rt.shutdown()


def test_trace_records_execution_order():
    model = Reversed()
    rt = LayerRuntime(model, dtype=torch.float32, prefetch_k=1, telemetry=False)
    x = torch.randn(2, 32)
    model(x)
    assert rt.trace_order == ["c", "b", "a"]
    model(x)
    assert rt.traced and rt.trace_order == ["c", "b", "a"]
    rt.shutdown()


def test_inference_and_backward():
    model = Seq(3)
    rt = LayerRuntime(model, dtype=torch.float32, inference_mode=True, telemetry=False)
    with torch.no_grad():
        model(torch.randn(2, 32))
        out = model(torch.randn(2, 32))
    assert rt.mode == "scheduled" and out.shape == (2, 32)
    rt.shutdown()

    model = Seq(3)
    ref = Seq(3)
    ref.load_state_dict(model.state_dict())
    rt = LayerRuntime(model, dtype=torch.float32, prefetch_k=1, telemetry=False)
    x = torch.randn(2, 32)
    for _ in range(2):
        xg = x.clone().requires_grad_(True)
        model(xg).sum().backward()
        assert xg.grad is not None
    xr = x.clone().requires_grad_(True)
    ref(xr).sum().backward()
    assert rt.mode == "scheduled"
    assert torch.allclose(xg.grad, xr.grad, atol=1e-6)
    rt.shutdown()


def test_shutdown_and_pool_reuse():
    model = Seq(3)
    rt = LayerRuntime(model, dtype=torch.float32, telemetry=False)
    model(torch.randn(2, 32))
    rt.shutdown()
    rt.shutdown()
    assert rt.mode == "shutdown"

    rt1 = LayerRuntime(Seq(3), dtype=torch.float32, telemetry=False)
    pool = rt1.shutdown_keep_pool()
    assert rt1.mode == "shutdown" and pool.stats()["total"] > 0
    model2 = Seq(3)
    rt2 = LayerRuntime(model2, dtype=torch.float32, telemetry=False, pool=pool)
    model2(torch.randn(2, 32))
    model2(torch.randn(2, 32))
    assert rt2.mode == "scheduled"
    rt2.shutdown()


def test_edge_cases():
    with pytest.raises(ValueError, match="No eligible layers"):
        LayerRuntime(nn.Sequential(nn.BatchNorm1d(32)), dtype=torch.float32)
    single = nn.Sequential(nn.Linear(32, 16))
    rt = LayerRuntime(single, dtype=torch.float32, telemetry=False)
    single(torch.randn(2, 32))
    single(torch.randn(2, 32))
    assert rt.num_layers == 1 and rt.mode == "scheduled"
    rt.shutdown()
    assert LayerRuntime(Shared(), dtype=torch.float32, telemetry=False).num_layers == 2


def test_top_level_api():
    m = Seq(4)
    assert stagehand.layer(m, dtype=torch.float32, telemetry=False) is m
    assert isinstance(m._stagehand_layer_runtime, LayerRuntime)
    for _ in range(3):
        assert m(torch.randn(2, 32)).shape == (2, 32)
    m._stagehand_layer_runtime.shutdown()
    w = Seq(3)
    assert stagehand.wrap(w, dtype=torch.float32, telemetry=False) is w
    w._stagehand_layer_runtime.shutdown()
    r = Seq(3)
    assert stagehand.Runtime(dtype=torch.float32, telemetry=False).layer(r) is r
    r._stagehand_layer_runtime.shutdown()


# ── config 1: the reference's CPU plumbing case ─────────────────────────


def test_config1_cpu_plumbing():
    """8 × Linear(4096, 4096) fp32 (W ~ N(0, .02), b = 0, fixed seed), bf16 storage,
    prefetch_k=3, inference: trace step then scheduled step."""
    from oracle.squareq import bf16_rne_bits

    torch.manual_seed(0)
    model = nn.Sequential(*[nn.Linear(4096, 4096) for _ in range(8)])
    with torch.no_grad():
        for lin in model:
            lin.weight.normal_(0, 0.02)
            lin.bias.zero_()
    want = [np.concatenate([bf16_rne_bits(lin.weight.detach().numpy().reshape(-1)),
                            bf16_rne_bits(lin.bias.detach().numpy())]) for lin in model]
    ref = nn.Sequential(*[nn.Linear(4096, 4096) for _ in range(8)])
    ref.load_state_dict(model.state_dict())
    ref = ref.to(torch.bfloat16)
    x = torch.randn(16, 4096).to(torch.bfloat16)  # the layer views are bf16, so the input is too
    m = stagehand.layer(model, dtype=torch.bfloat16, prefetch_k=3, inference_mode=True)
    rt = m._stagehand_layer_runtime
    assert (rt.config.pinned_slab_mb, rt.pool.num_slabs) == (64, 7)
    with torch.no_grad():
        y0, y1, yr = m(x), m(x), ref(x)
    assert rt.mode == "scheduled"
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))
    assert torch.equal(y0.view(torch.int16), yr.view(torch.int16))
    total = 0
    for i in range(8):
        buf = rt.residency.get_entry(str(i)).gpu_tensor
        got = buf.view(torch.int16).numpy().view(np.uint16)
        assert got.nbytes == 33_562_624
        assert np.array_equal(got, want[i])
        total += got.nbytes
    assert total == 268_500_992
    rt.shutdown()
