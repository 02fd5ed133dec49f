"""The reference's host staging ops, restated with the same torch CPU calls.

Test infrastructure and the reported CPU baseline only (see oracle/__init__.py).
These functions issue exactly the torch op sequence of the reference so that
timing them measures what the reference spends on the host per block:

* ``host_dequant_into`` — src/stagehand/scheduler.py:290-300:
  ``(q2d.to(f32) - zero_vec.unsqueeze(1)) * scale_vec.unsqueeze(1)``, then
  ``.to(bf16)`` and ``copy_`` into the slab at the layout offset;
* ``host_cast_into`` — src/stagehand/scheduler.py:181 / :1071:
  ``region.copy_(param.to(bf16).reshape(-1))``.
"""
from __future__ import annotations

from typing import Sequence

import torch

__all__ = ["host_dequant_into", "host_cast_into"]


def host_dequant_into(
    slab_u8: torch.Tensor,
    regions: Sequence[tuple[int, torch.Tensor, torch.Tensor, torch.Tensor, int, int]],
    dtype: torch.dtype = torch.bfloat16,
) -> None:
    """regions: (offset_bytes, qweight int8 2-D, scale f32, zero_point f32, out_dim, in_dim)."""
    elem = dtype.itemsize
    for offset_bytes, qweight, scale, zero_point, out_dim, in_flat in regions:
        nbytes = out_dim * in_flat * elem
        dst_region = slab_u8[offset_bytes: offset_bytes + nbytes]
        q2d = qweight.reshape(int(qweight.shape[0]), -1)
        q2d = q2d[:out_dim, :in_flat]
        scale_vec = scale.reshape(-1).to(dtype=torch.float32)[:out_dim]
        zero_vec = zero_point.reshape(-1).to(dtype=torch.float32)[:out_dim]
        dequant = (q2d.to(torch.float32) - zero_vec.unsqueeze(1)) * scale_vec.unsqueeze(1)
        dst_region.copy_(dequant.to(dtype=dtype).reshape(out_dim, in_flat).view(torch.uint8).reshape(-1))


def host_cast_into(
    slab_u8: torch.Tensor,
    regions: Sequence[tuple[int, torch.Tensor]],
    dtype: torch.dtype = torch.bfloat16,
) -> None:
    """regions: (offset_bytes, fp32 parameter tensor)."""
    elem = dtype.itemsize
    for offset_bytes, param in regions:
        nbytes = param.numel() * elem
        region = slab_u8[offset_bytes: offset_bytes + nbytes].view(dtype)
        region.copy_(param.data.to(dtype).reshape(-1))
