"""Every branch of the SquareQ block staging, end to end through the runtime.

The reference stages a SquareQ-backed block with ``_copy_squareq_backed_params_into_buffer``
(src/stagehand/scheduler.py:243-325). Besides the dequant of a well-formed layer it has
fallbacks: zero fill for a 0-d parameter, non-positive dimensions and short scale or
zero-point vectors; a weight whose layer lacks one of qweight/scale/zero_point, and any
parameter whose layer is missing or not a dict, falls through to the module branch, which
casts the live module parameter, or after eviction (size-0 data) its per-block CPU cache,
and otherwise zero-fills; a bias spec whose layer has no bias is zero-filled.

These tests build blocks that reach each branch, stage them through ``StagehandRuntime``
(the scheduler's ``before_block``), and compare the block buffer byte for byte with
``oracle.squareq.stage_squareq_block`` — on the GPU through the native loader and unpack
kernel, and on the CPU through the host staging path. A second load after an eviction,
with some module parameters emptied and one changed, checks the cache and the live reads.
The two module-branch fallbacks of a SquareQ weight (a layer without ``zero_point``, a layer
that is not a dict) are also compared directly with torch's cast of the module parameter, live
and then from the cache, independently of the oracle.
"""
from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest
import torch
from torch import nn

import stagehand_amd as stagehand
from oracle import squareq as oq
from stagehand_amd.config import StagehandConfig
from stagehand_amd.registry import SquareQParamSpec


class FallbackBlock(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.s0 = nn.Parameter(torch.tensor(0.5))      # 0-d, weight spec → zeros
        self.z0 = nn.Parameter(torch.zeros(0, 5))      # out_dim 0 → zeros (0 bytes)
        self.z1 = nn.Parameter(torch.zeros(3, 0))      # in_flat 0 → zeros (0 bytes)
        self.a = nn.Linear(96, 64)    # dequant with padded_in 100 and non-zero zero points; bias cast
        self.b = nn.Linear(64, 40)    # scale vector shorter than out → zeros; bias cast
        self.c = nn.Linear(64, 40)    # zero-point vector shorter than out → zeros; layer has no bias → zeros
        self.d = nn.Linear(32, 24)    # layer without zero_point → module branch (live); bias module
        self.e = nn.Linear(32, 24)    # layer without scale, not a module param → zeros; bias: layer missing → module
        self.f = nn.Linear(16, 8)     # layer is not a dict → module branch; bias: no spec, no module → zeros
        self.norm = nn.LayerNorm(32)  # module-resident


class FallbackStack(nn.Module):
    def __init__(self, n: int = 2) -> None:
        super().__init__()
        self.blocks = nn.ModuleList(FallbackBlock() for _ in range(n))


MODULE_NAMES = ("d.weight", "d.bias", "e.bias", "f.weight", "norm.weight", "norm.bias")


def _payload(n_blocks: int, seed: int = 3) -> dict:
    g = torch.Generator().manual_seed(seed)

    def q(o, i):
        return torch.randint(-127, 128, (o, i), dtype=torch.int8, generator=g)

    def s(n):
        return torch.exp(torch.randn(n, generator=g) * 0.5 - 6.0)

    layers, manifest = {}, []
    for bi in range(n_blocks):
        p = f"blocks.{bi}"
        layers[f"{p}.a"] = {"qweight": q(64, 100), "scale": s(64), "zero_point": torch.randn(64, generator=g) * 3,
                            "bias": torch.randn(64, generator=g) * 0.1}
        layers[f"{p}.b"] = {"qweight": q(40, 64), "scale": s(30), "zero_point": torch.zeros(40),
                            "bias": torch.randn(40, generator=g) * 0.1}
        layers[f"{p}.c"] = {"qweight": q(40, 64), "scale": s(40), "zero_point": torch.zeros(20)}
        layers[f"{p}.d"] = {"qweight": q(24, 32), "scale": s(24)}
        layers[f"{p}.e"] = {"qweight": q(24, 32), "zero_point": torch.zeros(24)}
        layers[f"{p}.f"] = torch.ones(3)
        manifest.append({"name": f"{p}.a", "out": 64, "inp": 96, "padded_in": 100, "has_bias": True})
    return {"manifest": {"layout": "rowwise_sym_int8", "layers": manifest}, "layers": layers}


def _specs(bid: str) -> dict[str, tuple[str, str]]:
    """param → (layer, kind) for the crafted block."""
    return {
        "s0": (f"{bid}.a", "weight"), "z0": (f"{bid}.a", "weight"), "z1": (f"{bid}.a", "weight"),
        "a.weight": (f"{bid}.a", "weight"), "a.bias": (f"{bid}.a", "bias"),
        "b.weight": (f"{bid}.b", "weight"), "b.bias": (f"{bid}.b", "bias"),
        "c.weight": (f"{bid}.c", "weight"), "c.bias": (f"{bid}.c", "bias"),
        "d.weight": (f"{bid}.d", "weight"),
        "e.weight": (f"{bid}.e", "weight"), "e.bias": (f"{bid}.missing", "bias"),
        "f.weight": (f"{bid}.f", "weight"),
    }


def _np_layers(layers: dict) -> dict:
    out = {}
    for k, v in layers.items():
        out[k] = {kk: vv.numpy() for kk, vv in v.items()} if isinstance(v, dict) else v.numpy()
    return out


def _module_values(block: nn.Module) -> dict[str, np.ndarray | None]:
    """The module's parameters as the staging sees them (a size-0 array once evicted)."""
    return {name: p.data.float().cpu().numpy() for name, p in block.named_parameters()}


def _buffer_bytes(rt, bid: str) -> np.ndarray:
    buf = rt.residency.get_entry(bid).gpu_tensor
    return buf.detach().contiguous().view(torch.uint8).cpu().numpy()


def _run(tmp_path) -> None:
    n = 2
    torch.manual_seed(11)
    model = FallbackStack(n)
    for p in model.parameters():
        p.requires_grad_(False)
    payload = _payload(n)
    path = tmp_path / "fallbacks.fpk"
    torch.save(payload, path)
    cfg = StagehandConfig(pinned_pool_mb=16, pinned_slab_mb=1, vram_high_watermark_mb=200000,
                          vram_low_watermark_mb=100000, prefetch_window_blocks=1, telemetry_enabled=False,
                          nan_inf_check=False, strict_bf16=False)
    rt = stagehand.StagehandRuntime(model, cfg, block_pattern=r"^blocks\.\d+$", dtype=torch.bfloat16,
                                    inference_mode=True)
    assert rt.convert_registry_to_file_backed(str(path)) == 2 * n  # a.weight and a.bias of each block
    np_layers = _np_layers(payload["layers"])
    layouts, specs_np, caches = {}, {}, {}
    for bi in range(n):
        bid = f"blocks.{bi}"
        entry = rt.registry.get(bid)
        assert entry.squareq_backed and entry.source_format == "squareq_bp8"
        manifest = {f"{bid}.a": (64, 96, 100)}
        specs, specs_np[bid] = [], {}
        for pname, (layer, kind) in _specs(bid).items():
            o, i, pad = manifest.get(layer, (0, 0, 0))
            specs.append(SquareQParamSpec(pname, layer, kind, o, i, pad))
            specs_np[bid][pname] = oq.SquareQSpec(pname, layer, kind, o, i, pad)
        rt.registry._entries[bid] = replace(entry, squareq_param_specs=tuple(specs), module_param_names=MODULE_NAMES)
        layouts[bid] = [oq.LayoutEntry(name, shape, "bfloat16", off, numel)
                        for name, shape, _dt, off, numel in entry.param_layout]
        caches[bid] = {}
    rt._scheduler.refresh_registry_snapshot()
    sched = rt._scheduler

    def region(bid: str, got: np.ndarray, name: str) -> np.ndarray:
        e = next(e for e in layouts[bid] if e.name == name)
        return got[e.offset:e.offset + e.nbytes].view(np.uint16)

    def torch_bf16(t: torch.Tensor) -> np.ndarray:
        """The reference's module-branch cast (scheduler.py:310-322: ``param.data.to(dtype)``)."""
        return t.detach().cpu().to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16).reshape(-1)

    # What the module branch must copy, in closed form: d.weight's layer has no zero_point and f's
    # layer is not a dict, so both take the module parameter as it is when the block is staged,
    # then (evicted to size 0) the value the block's first staging cached.
    first = {bi: {k: getattr(getattr(model.blocks[bi], k.split(".")[0]), k.split(".")[1]).detach().clone()
                  for k in ("d.weight", "f.weight", "e.bias")} for bi in range(n)}
    expect_module = {0: {bi: dict(first[bi]) for bi in range(n)}}

    def load_and_check(step: int) -> None:
        rt.begin_step(step)
        for bi in range(n):
            bid = f"blocks.{bi}"
            block = model.blocks[bi]
            want = oq.stage_squareq_block(layouts[bid], specs_np[bid], set(MODULE_NAMES), _module_values(block),
                                          np_layers, caches[bid])
            sched.before_block(bid)
            got = _buffer_bytes(rt, bid)
            assert got.size == len(want), (step, bid)
            bad = np.flatnonzero(got != np.frombuffer(bytes(want), np.uint8))
            if bad.size:
                at = int(bad[0])
                name = next(e.name for e in layouts[bid] if e.offset <= at < e.offset + e.nbytes)
                raise AssertionError(f"step {step} {bid}: byte {at} ({name}) differs from the oracle")
            for name, value in expect_module[step][bi].items():
                assert np.array_equal(region(bid, got, name), torch_bf16(value)), (step, bid, name)
            sched.after_block(bid)
        rt.end_step()

    load_and_check(0)
    # the branches did what they should (the oracle agrees with the closed forms too)
    blk0 = model.blocks[0]
    assert torch.count_nonzero(blk0.b.weight.float()) == 0 and torch.count_nonzero(blk0.c.weight.float()) == 0
    assert torch.count_nonzero(blk0.c.bias.float()) == 0 and torch.count_nonzero(blk0.e.weight.float()) == 0
    assert torch.count_nonzero(blk0.f.bias.float()) == 0 and float(blk0.s0.float()) == 0.0
    for bi in range(n):
        sched._evict_block(f"blocks.{bi}")
    g = torch.Generator().manual_seed(5)
    for bi in range(n):
        blk = model.blocks[bi]
        blk.e.bias.data = torch.empty(0)            # evicted: the block's cache holds its first value
        blk.f.weight.data = torch.empty(0)
        blk.d.weight.data = torch.randn(24, 32, generator=g)  # live: read as it is now
    expect_module[1] = {bi: {"d.weight": model.blocks[bi].d.weight.data.clone(), "f.weight": first[bi]["f.weight"],
                             "e.bias": first[bi]["e.bias"]} for bi in range(n)}
    load_and_check(1)
    rt.shutdown()


@pytest.mark.gpu
def test_squareq_fallback_branches_on_the_device(tmp_path):
    assert torch.cuda.is_available()
    _run(tmp_path)


def test_squareq_fallback_branches_on_the_host(tmp_path):
    if torch.cuda.is_available():
        pytest.skip("the host staging path runs where there is no GPU")
    _run(tmp_path)
