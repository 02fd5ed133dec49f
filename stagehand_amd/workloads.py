"""Synthetic workloads of the benchmark configurations (seeded, no downloads).

``config2_*`` builds the dequant/unpack microbenchmark: a packed slab of 128
tensors cycling through 3072x3072, 3072x12288, 12288x3072, 3072x1 and 1000x77,
int8 values uniform in [-127, 127], per-output-row fp32 scales
exp(N(-6, 0.5)); the fp32 variant holds N(0, 0.02) values of the same shapes.
Source regions are packed back to back with no padding, exactly as the
reference lays out block buffers (src/stagehand/scheduler.py:148-165), so the
int8 regions after each 1000x77 tensor start 8 bytes off a 16-byte boundary.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from stagehand_amd.unpack import KIND_F32_BF16, KIND_I8_ROWSCALE_BF16, make_descs

__all__ = ["CONFIG2_SHAPES", "Region", "config2_regions", "config2_descs", "config2_device_inputs"]

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
