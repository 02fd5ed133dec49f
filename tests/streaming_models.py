"""Small models and SquareQ/safetensors writers shared by the streaming tests."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch
from torch import nn


class TinyBlock(nn.Module):
    """A transformer-ish block: norm + two Linears (+ bias) + a GELU."""

    def __init__(self, hidden: int = 64, mlp: int = 4) -> None:
        super().__init__()
        self.norm = nn.LayerNorm(hidden)
        self.fc1 = nn.Linear(hidden, hidden * mlp)
        self.fc2 = nn.Linear(hidden * mlp, hidden)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return x + self.fc2(torch.nn.functional.gelu(self.fc1(self.norm(x))))


class TinyStack(nn.Module):
    def __init__(self, n: int = 6, hidden: int = 64, mlp: int = 4) -> None:
        super().__init__()
        self.blocks = nn.ModuleList(TinyBlock(hidden, mlp) for _ in range(n))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        for b in self.blocks:
            x = b(x)
        return x


def init_(model: nn.Module, seed: int = 0) -> nn.Module:
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("norm.weight"):
                p.copy_(1.0 + 0.1 * torch.randn(p.shape, generator=g))
            else:
                p.copy_(0.05 * torch.randn(p.shape, generator=g))
    return model


def squareq_payload(model: TinyStack, seed: int = 1, padded: int = 0, with_zp: bool = False) -> dict:
    """Quantised layers for every Linear of every block: q ~ U{-127..127}, s = exp(N(-6, .5))."""
    g = torch.Generator().manual_seed(seed)
    layers, manifest = {}, []
    for bi, blk in enumerate(model.blocks):
        for lname in ("fc1", "fc2"):
            lin = getattr(blk, lname)
            out_f, in_f = lin.weight.shape
            pad_in = in_f + padded
            q = torch.randint(-127, 128, (out_f, pad_in), dtype=torch.int8, generator=g)
            s = torch.exp(torch.randn(out_f, generator=g) * 0.5 - 6.0)
            z = (torch.randn(out_f, generator=g) if with_zp else torch.zeros(out_f))
            name = f"blocks.{bi}.{lname}"
            layers[name] = {"qweight": q, "scale": s, "zero_point": z, "bias": torch.randn(out_f, generator=g) * 0.1}
            manifest.append({"name": name, "out": out_f, "inp": in_f, "padded_in": pad_in, "has_bias": True})
    return {"manifest": {"layout": "rowwise_sym_int8", "layers": manifest}, "layers": layers}


def expected_squareq_weight(layer: dict, out_f: int, in_f: int, dtype: torch.dtype) -> torch.Tensor:
    """Torch CPU restatement of src/stagehand/scheduler.py:290-300 for one weight."""
    q2d = layer["qweight"].reshape(layer["qweight"].shape[0], -1)[:out_f, :in_f]
    deq = (q2d.to(torch.float32) - layer["zero_point"].reshape(-1)[:out_f].unsqueeze(1)) * layer["scale"].reshape(-1)[:out_f].unsqueeze(1)
    return deq.to(dtype)


def save_safetensors(model: nn.Module, path: Path, dtype: torch.dtype) -> None:
    from safetensors.torch import save_file

    save_file({k: v.detach().to(dtype).contiguous() for k, v in model.state_dict().items()}, str(path))
