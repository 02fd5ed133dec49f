"""Numeric checks on block outputs (the interface of src/stagehand/guards.py:34-161).

Not on the data path: the scheduler calls ``check_output`` after a block's
compute when ``nan_inf_check`` is on.

* ``check_output`` counts NaN and Inf elements (0, 0 when disabled);
* ``check_dtype`` raises DtypeMismatchError in strict mode when a tensor's
  dtype is not the expected one;
* ``check_promotion`` raises when an output dtype ranks above its input
  dtype (fp8 < bf16 = fp16 < fp32 < fp64; unknown dtypes never raise).
"""
from __future__ import annotations

import logging

import torch

from stagehand_amd.errors import DtypeMismatchError

__all__ = ["NumericGuard"]

log = logging.getLogger(__name__)

_RANK: dict[torch.dtype, int] = {torch.float8_e5m2: 0, torch.float8_e4m3fn: 0, torch.bfloat16: 1, torch.float16: 1,
                                 torch.float32: 2, torch.float64: 3}


class NumericGuard:
    def __init__(self, strict_bf16: bool = True, fail_on_dtype_promotion: bool = True, nan_inf_check: bool = True) -> None:
        self._strict_bf16 = strict_bf16
        self._fail_on_dtype_promotion = fail_on_dtype_promotion
        self._nan_inf_check = nan_inf_check

    def check_dtype(self, tensor: torch.Tensor, expected_dtype: torch.dtype, context: str) -> None:
        if self._strict_bf16 and tensor.dtype != expected_dtype:
            raise DtypeMismatchError(f"[{context}] expected dtype {expected_dtype}, got {tensor.dtype}")

    def check_output(self, tensor: torch.Tensor, block_id: str, step: int) -> tuple[int, int]:
        if not self._nan_inf_check or bool(torch.isfinite(tensor).all()):
            return 0, 0
        nan_count = int(torch.isnan(tensor).sum().item())
        inf_count = int(torch.isinf(tensor).sum().item())
        log.warning("non-finite output of block %r at step %d: %d NaN, %d Inf (shape %s)", block_id, step,
                    nan_count, inf_count, list(tensor.shape))
        return nan_count, inf_count

    def check_promotion(self, input_dtype: torch.dtype, output_dtype: torch.dtype, context: str) -> None:
        if not self._fail_on_dtype_promotion:
            return
        src, dst = _RANK.get(input_dtype, -1), _RANK.get(output_dtype, -1)
        if src >= 0 and dst >= 0 and dst > src:
            raise DtypeMismatchError(f"[{context}] dtype promotion {input_dtype} -> {output_dtype}")
