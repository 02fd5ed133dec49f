"""Synthetic workloads of the benchmark configurations (seeded, no downloads).

Used by ``bench.py`` and the tests; not part of the ``stagehand_amd`` package.

``config2_*`` builds the dequant/unpack microbenchmark: a packed slab of 128
tensors cycling through 3072x3072, 3072x12288, 12288x3072, 3072x1 and 1000x77,
int8 values uniform in [-127, 127], per-output-row fp32 scales
exp(N(-6, 0.5)); the fp32 variant holds N(0, 0.02) values of the same shapes.
Source regions are packed back to back with no padding, exactly as the
reference lays out block buffers (src/stagehand/scheduler.py:148-165), so the
int8 regions after each 1000x77 tensor start 8 bytes off a 16-byte boundary.
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

from stagehand_amd.unpack import KIND_F32_BF16, KIND_I8_ROWSCALE_BF16, make_descs

__all__ = ["CONFIG2_SHAPES", "Region", "config2_regions", "config2_descs", "config2_device_inputs", "FluxStyleDiT",
           "TrainDiT", "write_dit_squareq", "write_dit_safetensors_sharded"]

CONFIG2_SHAPES: tuple[tuple[int, int], ...] = ((3072, 3072), (3072, 12288), (12288, 3072), (3072, 1), (1000, 77))


@dataclass(frozen=True)
class Region:
    index: int
    rows: int
    cols: int
    elem_off: int   # element offset of the region in the packed slab
    scale_off: int  # index of its first row scale

    @property
    def numel(self) -> int:
        return self.rows * self.cols


def config2_regions(n_tensors: int = 128, shapes=CONFIG2_SHAPES) -> list[Region]:
    regions = []
    elem = 0
    rows_total = 0
    for i in range(n_tensors):
        r, c = shapes[i % len(shapes)]
        regions.append(Region(i, r, c, elem, rows_total))
        elem += r * c
        rows_total += r
    return regions


def config2_descs(regions: list[Region], variant: str = "dequant") -> np.ndarray:
    """Descriptor table: int8 (1 B) or fp32 (4 B) source at elem_off, bf16 destination at 2*elem_off."""
    if variant == "dequant":
        return make_descs((KIND_I8_ROWSCALE_BF16, g.elem_off, 2 * g.elem_off, g.rows, g.cols, 0, g.scale_off)
                          for g in regions)
    if variant == "cast":
        return make_descs((KIND_F32_BF16, 4 * g.elem_off, 2 * g.elem_off, 1, g.numel, 0, 0) for g in regions)
    raise ValueError(variant)


def config2_device_inputs(regions: list[Region], variant: str, seed: int, device: str = "cuda"):
    """Generates the source slab (and scales) directly on the device with a seeded generator."""
    n = sum(g.numel for g in regions)
    rows = sum(g.rows for g in regions)
    gen = torch.Generator(device=device).manual_seed(seed)
    if variant == "dequant":
        src = torch.randint(-127, 128, (n,), dtype=torch.int8, device=device, generator=gen)
        scales = torch.exp(torch.randn(rows, device=device, generator=gen) * 0.5 - 6.0).to(torch.float32)
        return src, scales
    if variant == "cast":
        src = torch.randn(n, device=device, generator=gen, dtype=torch.float32) * 0.02
        return src, None
    raise ValueError(variant)


# ── Flux-style DiT (configs 3-5) ─────────────────────────────────────────────

import math as _math

from torch import nn as _nn
from torch.nn import functional as _F


class _QKNorm(_nn.Module):
    def __init__(self, head_dim: int) -> None:
        super().__init__()
        self.query_norm = _nn.RMSNorm(head_dim, eps=1e-6)
        self.key_norm = _nn.RMSNorm(head_dim, eps=1e-6)


def _attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """(B, H, S, D) scaled dot-product attention on the fused (flash) kernel only."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        return _F.scaled_dot_product_attention(q.contiguous(), k.contiguous(), v.contiguous())


def _split_heads(x: torch.Tensor, heads: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    b, s, three_h = x.shape
    d = three_h // (3 * heads)
    qkv = x.view(b, s, 3, heads, d).permute(2, 0, 3, 1, 4)
    return qkv[0], qkv[1], qkv[2]


class DoubleStreamBlock(_nn.Module):
    """Image and text streams with joint attention (Flux double-stream layout)."""

    def __init__(self, hidden: int, heads: int, mlp_ratio: float) -> None:
        super().__init__()
        mlp = int(hidden * mlp_ratio)
        self.heads = heads
        for side in ("img", "txt"):
            setattr(self, f"{side}_mod", _nn.Linear(hidden, 6 * hidden))
            setattr(self, f"{side}_qkv", _nn.Linear(hidden, 3 * hidden))
            setattr(self, f"{side}_qk_norm", _QKNorm(hidden // heads))
            setattr(self, f"{side}_proj", _nn.Linear(hidden, hidden))
            setattr(self, f"{side}_mlp", _nn.Sequential(_nn.Linear(hidden, mlp), _nn.GELU(approximate="tanh"),
                                                         _nn.Linear(mlp, hidden)))

    def forward(self, img: torch.Tensor, txt: torch.Tensor, vec: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        h = img.shape[-1]
        sv = _F.silu(vec)[:, None, :]
        im = self.img_mod(sv).chunk(6, dim=-1)
        tm = self.txt_mod(sv).chunk(6, dim=-1)
        img_n = _F.layer_norm(img, (h,), eps=1e-6) * (1 + im[1]) + im[0]
        txt_n = _F.layer_norm(txt, (h,), eps=1e-6) * (1 + tm[1]) + tm[0]
        iq, ik, iv = _split_heads(self.img_qkv(img_n), self.heads)
        tq, tk, tv = _split_heads(self.txt_qkv(txt_n), self.heads)
        iq, ik = self.img_qk_norm.query_norm(iq), self.img_qk_norm.key_norm(ik)
        tq, tk = self.txt_qk_norm.query_norm(tq), self.txt_qk_norm.key_norm(tk)
        q, k, v = torch.cat([tq, iq], 2), torch.cat([tk, ik], 2), torch.cat([tv, iv], 2)
        attn = _attention(q, k, v).permute(0, 2, 1, 3).reshape(img.shape[0], -1, h)
        t_attn, i_attn = attn[:, : txt.shape[1]], attn[:, txt.shape[1]:]
        img = img + im[2] * self.img_proj(i_attn)
        img = img + im[5] * self.img_mlp(_F.layer_norm(img, (h,), eps=1e-6) * (1 + im[4]) + im[3])
        txt = txt + tm[2] * self.txt_proj(t_attn)
        txt = txt + tm[5] * self.txt_mlp(_F.layer_norm(txt, (h,), eps=1e-6) * (1 + tm[4]) + tm[3])
        return img, txt


class SingleStreamBlock(_nn.Module):
    """Fused QKV+MLP-in projection and fused output projection (Flux single-stream layout)."""

    def __init__(self, hidden: int, heads: int, mlp_ratio: float) -> None:
        super().__init__()
        self.hidden, self.heads, self.mlp = hidden, heads, int(hidden * mlp_ratio)
        self.linear1 = _nn.Linear(hidden, 3 * hidden + self.mlp)
        self.linear2 = _nn.Linear(hidden + self.mlp, hidden)
        self.qk_norm = _QKNorm(hidden // heads)
        self.modulation = _nn.Linear(hidden, 3 * hidden)

    def forward(self, x: torch.Tensor, vec: torch.Tensor) -> torch.Tensor:
        h = self.hidden
        shift, scale, gate = self.modulation(_F.silu(vec)[:, None, :]).chunk(3, dim=-1)
        xn = _F.layer_norm(x, (h,), eps=1e-6) * (1 + scale) + shift
        qkv, mlp_in = torch.split(self.linear1(xn), [3 * h, self.mlp], dim=-1)
        q, k, v = _split_heads(qkv, self.heads)
        q, k = self.qk_norm.query_norm(q), self.qk_norm.key_norm(k)
        attn = _attention(q, k, v).permute(0, 2, 1, 3).reshape(x.shape[0], -1, h)
        return x + gate * self.linear2(torch.cat([attn, _F.gelu(mlp_in, approximate="tanh")], dim=-1))


class FluxStyleDiT(_nn.Module):
    """19 double-stream + 38 single-stream blocks, hidden 3072, 24 heads, MLP ratio 4 by default
    (11.84 B block parameters). Only the blocks are built: the benchmark feeds
    latent / text token activations and a conditioning vector directly."""

    def __init__(self, depth_double: int = 19, depth_single: int = 38, hidden: int = 3072, heads: int = 24,
                 mlp_ratio: float = 4.0) -> None:
        super().__init__()
        self.double_blocks = _nn.ModuleList(DoubleStreamBlock(hidden, heads, mlp_ratio) for _ in range(depth_double))
        self.single_blocks = _nn.ModuleList(SingleStreamBlock(hidden, heads, mlp_ratio) for _ in range(depth_single))

    def forward(self, img: torch.Tensor, txt: torch.Tensor, vec: torch.Tensor) -> torch.Tensor:
        for blk in self.double_blocks:
            img, txt = blk(img, txt, vec)
        x = torch.cat([txt, img], dim=1)
        for blk in self.single_blocks:
            x = blk(x, vec)
        return x[:, txt.shape[1]:]


DIT_BLOCK_PATTERN = r"^(double_blocks|single_blocks)\.\d+$"


def dit_linear_layers(model: _nn.Module) -> list[tuple[str, _nn.Linear]]:
    return [(n, m) for n, m in model.named_modules() if isinstance(m, _nn.Linear)]


def dit_forward_flops(model: FluxStyleDiT, img_tokens: int, txt_tokens: int) -> float:
    """Matmul FLOPs of one forward (2 per multiply-add; attention score and value products included)."""
    flops = 0.0
    for name, lin in dit_linear_layers(model):
        tokens = img_tokens if ".img_" in name else txt_tokens if ".txt_" in name else img_tokens + txt_tokens
        if name.endswith("_mod") or name.endswith("modulation"):
            tokens = 1
        flops += 2.0 * tokens * lin.in_features * lin.out_features
    s = img_tokens + txt_tokens
    for blk in list(model.double_blocks) + list(model.single_blocks):
        hidden = blk.img_proj.in_features if isinstance(blk, DoubleStreamBlock) else blk.hidden
        flops += 2 * 2.0 * s * s * hidden
    return flops


def materialize_norms_(model: _nn.Module, device: str = "cpu") -> None:
    """Gives a meta-device model real RMSNorm weights (ones); everything else stays meta."""
    for mod in model.modules():
        if isinstance(mod, _nn.RMSNorm) and mod.weight is not None:
            mod.weight = _nn.Parameter(torch.ones(mod.weight.shape, device=device), requires_grad=False)


# ── training DiT (config 5) ──────────────────────────────────────────────────


class LoRALinear(_nn.Module):
    """A frozen base Linear plus a trainable rank-r update: y = base(x) + (x Aᵀ) Bᵀ,
    A ~ N(0, 0.01), B = 0 (so the adapter starts as the identity update)."""

    def __init__(self, in_features: int, out_features: int, rank: int, bias: bool = True) -> None:
        super().__init__()
        self.base = _nn.Linear(in_features, out_features, bias=bias)
        self.lora_A = _nn.Parameter(torch.empty(rank, in_features))
        self.lora_B = _nn.Parameter(torch.zeros(out_features, rank))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.base(x) + _F.linear(_F.linear(x, self.lora_A), self.lora_B)


class _Attn(_nn.Module):
    def __init__(self, hidden: int, rank: int | None) -> None:
        super().__init__()
        make = (lambda: LoRALinear(hidden, hidden, rank)) if rank else (lambda: _nn.Linear(hidden, hidden))
        self.q, self.k, self.v, self.o = make(), make(), make(), make()


def _heads(x: torch.Tensor, heads: int) -> torch.Tensor:
    b, s, h = x.shape
    return x.view(b, s, heads, h // heads).transpose(1, 2)


class TrainBlock(_nn.Module):
    """WAN-style block: adaLN modulation, self-attention (LoRA on q/k/v/o),
    cross-attention over a conditioning sequence, GELU MLP — 22·h² weights."""

    def __init__(self, hidden: int, heads: int, mlp_ratio: float, rank: int) -> None:
        super().__init__()
        self.heads = heads
        self.modulation = _nn.Linear(hidden, 6 * hidden)
        self.self_attn = _Attn(hidden, rank)
        self.cross_attn = _Attn(hidden, None)
        mlp = int(hidden * mlp_ratio)
        self.ffn = _nn.Sequential(_nn.Linear(hidden, mlp), _nn.GELU(approximate="tanh"), _nn.Linear(mlp, hidden))

    def forward(self, x: torch.Tensor, ctx: torch.Tensor, vec: torch.Tensor) -> torch.Tensor:
        h, nh = x.shape[-1], self.heads
        m = self.modulation(_F.silu(vec)[:, None, :]).chunk(6, dim=-1)
        xn = _F.layer_norm(x, (h,), eps=1e-6) * (1 + m[1]) + m[0]
        sa = self.self_attn
        a = _attention(_heads(sa.q(xn), nh), _heads(sa.k(xn), nh), _heads(sa.v(xn), nh))
        x = x + m[2] * sa.o(a.transpose(1, 2).reshape(x.shape))
        ca = self.cross_attn
        xn = _F.layer_norm(x, (h,), eps=1e-6)
        a = _attention(_heads(ca.q(xn), nh), _heads(ca.k(ctx), nh), _heads(ca.v(ctx), nh))
        x = x + ca.o(a.transpose(1, 2).reshape(x.shape))
        return x + m[5] * self.ffn(_F.layer_norm(x, (h,), eps=1e-6) * (1 + m[4]) + m[3])


class TrainDiT(_nn.Module):
    """48 blocks, hidden 4096, 32 heads, MLP ratio 4, LoRA rank 32 on the self-attention
    projections by default (17.7 B frozen block weights, 50 M trainable). Blocks are
    recomputed in the backward pass (activation checkpointing) when ``checkpoint``."""

    def __init__(self, depth: int = 48, hidden: int = 4096, heads: int = 32, mlp_ratio: float = 4.0, rank: int = 32,
                 checkpoint: bool = True) -> None:
        super().__init__()
        self.checkpoint = checkpoint
        self.blocks = _nn.ModuleList(TrainBlock(hidden, heads, mlp_ratio, rank) for _ in range(depth))

    def forward(self, x: torch.Tensor, ctx: torch.Tensor, vec: torch.Tensor) -> torch.Tensor:
        from torch.utils.checkpoint import checkpoint

        for blk in self.blocks:
            if self.checkpoint and torch.is_grad_enabled():
                x = checkpoint(blk, x, ctx, vec, use_reentrant=False)
            else:
                x = blk(x, ctx, vec)
        return x


TRAIN_BLOCK_PATTERN = r"^blocks\.\d+$"


def init_train_dit_(model: TrainDiT, seed: int, device: str = "cpu") -> TrainDiT:
    """bf16 weights: base N(0, 0.02), LoRA A N(0, 0.01), LoRA B 0 (drawn on ``device`` with a
    seeded generator, then stored in host memory); base weights frozen, LoRA trainable."""
    g = torch.Generator(device=device).manual_seed(seed)
    for mod in model.modules():
        for name, prm in list(mod.named_parameters(recurse=False)):
            if isinstance(mod, LoRALinear) and name == "lora_B":
                t = torch.zeros(prm.shape, dtype=torch.bfloat16)
            else:
                std = 0.01 if (isinstance(mod, LoRALinear) and name == "lora_A") else 0.02
                t = (torch.randn(prm.shape, device=device, generator=g) * std).to(torch.bfloat16).cpu()
            trainable = isinstance(mod, LoRALinear)
            setattr(mod, name, _nn.Parameter(t, requires_grad=trainable))
    return model


# ── weight files of the DiT configurations ──────────────────────────────────


def write_dit_squareq(model, path: Path, seed: int) -> dict:
    """SquareQ v1 slab (torch.save payload) for every block Linear of ``model``:
    int8 weights U{-127..127}, fp32 per-row scales exp(N(-6, 0.5)), zero points 0,
    bf16 biases N(0, 0.02); generated on the device, written through host memory."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    layers, manifest = {}, []
    for name, lin in dit_linear_layers(model):
        o, i = lin.out_features, lin.in_features
        q = torch.randint(-127, 128, (o, i), dtype=torch.int8, device="cuda", generator=g).cpu()
        sc = torch.exp(torch.randn(o, device="cuda", generator=g) * 0.5 - 6.0).cpu()
        b = (torch.randn(o, device="cuda", generator=g) * 0.02).to(torch.bfloat16).cpu()
        layers[name] = {"qweight": q, "scale": sc, "zero_point": torch.zeros(o), "bias": b}
        manifest.append({"name": name, "out": o, "inp": i, "padded_in": i, "has_bias": True})
    torch.save({"manifest": {"layout": "rowwise_sym_int8", "layers": manifest}, "layers": layers}, str(path))
    return {n: l for n, l in layers.items()}


def write_dit_safetensors_sharded(model, directory: Path, seed: int) -> int:
    """bf16 N(0, 0.02) weights, one safetensors shard per block + the index JSON."""
    from safetensors.torch import save_file

    directory.mkdir(parents=True, exist_ok=True)
    g = torch.Generator(device="cuda").manual_seed(seed)
    weight_map, total = {}, 0
    blocks = [(f"double_blocks.{i}", b) for i, b in enumerate(model.double_blocks)] + \
             [(f"single_blocks.{i}", b) for i, b in enumerate(model.single_blocks)]
    for bname, blk in blocks:
        tensors = {}
        for pname, prm in blk.named_parameters():
            key = f"{bname}.{pname}"
            if pname.endswith("norm.weight"):
                tensors[key] = torch.ones(prm.shape, dtype=torch.bfloat16)
            else:
                tensors[key] = (torch.randn(prm.shape, device="cuda", generator=g) * 0.02).to(torch.bfloat16).cpu()
            total += tensors[key].numel() * 2
        shard = f"{bname}.safetensors"
        save_file(tensors, str(directory / shard))
        weight_map.update({k: shard for k in tensors})
    (directory / "diffusion_pytorch_model.safetensors.index.json").write_text(
        json.dumps({"metadata": {"total_size": total}, "weight_map": weight_map}))
    return total
