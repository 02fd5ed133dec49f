"""Numeric checks on block outputs (the interface of src/stagehand/guards.py:34-161).

Not on the data path: the scheduler calls ``check_output`` after a block's
compute when ``nan_inf_check`` is on. Counts NaN/Inf elements; with
``strict_bf16`` a floating output that is not bf16 is counted as a dtype
promotion and, with ``fail_on_dtype_promotion``, raises DtypeMismatchError.
"""
from __future__ import annotations

import torch

from stagehand_amd.errors import DtypeMismatchError

__all__ = ["NumericGuard"]


class NumericGuard:
    def __init__(self, strict_bf16: bool = True, fail_on_dtype_promotion: bool = True, nan_inf_check: bool = True) -> None:
        self.strict_bf16 = strict_bf16
        self.fail_on_dtype_promotion = fail_on_dtype_promotion
        self.nan_inf_check = nan_inf_check
        self.promotions = 0

    def check_output(self, tensor: torch.Tensor, block_id: str, step: int) -> tuple[int, int]:
        if self.strict_bf16 and tensor.is_floating_point() and tensor.dtype != torch.bfloat16:
            self.promotions += 1
            if self.fail_on_dtype_promotion:
                raise DtypeMismatchError(f"block {block_id!r} produced {tensor.dtype} at step {step} (strict bf16)")
        if not self.nan_inf_check or not tensor.is_floating_point():
            return 0, 0
        return int(torch.isnan(tensor).sum().item()), int(torch.isinf(tensor).sum().item())
