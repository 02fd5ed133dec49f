"""numpy restatement of the reference's host staging arithmetic (oracle only).

See ``oracle/__init__.py``: test infrastructure, never imported by the product.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Mapping, Sequence

import numpy as np

__all__ = [
    "bf16_rne_bits",
    "bf16_bits_to_f32",
    "dequant_rows",
    "cast_f32_bf16",
    "LayoutEntry",
    "build_param_layout",
    "flatten_params",
    "stage_squareq_block",
    "SquareQSpec",
]

ITEMSIZE = {"bfloat16": 2, "float16": 2, "float32": 4, "int8": 1, "uint8": 1}


def bf16_rne_bits(x: np.ndarray) -> np.ndarray:
    """fp32 → bf16 bit patterns, round to nearest even; NaN → 0xFFFF.

    Follows torch's CPU float→bfloat16 conversion, which the reference invokes
    at src/stagehand/scheduler.py:181, 230, 300, 305 and 1071
    (``.to(torch.bfloat16)`` / ``copy_`` into a bf16 view). For non-NaN input
    this is c10's round_to_nearest_even, (u + 0x7FFF + ((u >> 16) & 1)) >> 16;
    torch's vectorised CPU path writes 0xFFFF for every NaN.
    """
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    r[np.isnan(f)] = 0xFFFF
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    """Exact widening of bf16 bit patterns to fp32."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def dequant_rows(
    qweight: np.ndarray,
    scale: np.ndarray,
    zero_point: np.ndarray | None,
    out_dim: int,
    in_dim: int,
    out: str = "bfloat16",
) -> np.ndarray:
    """SquareQ row-wise dequant of one weight, src/stagehand/scheduler.py:285-300.

    ``q2d = qweight.reshape(rows_q, -1)[:out, :in]`` (drops padded_in columns,
    :290-291); ``scale_vec``/``zero_vec`` are the first ``out`` fp32 entries
    (:293-294); the value is ``(f32(q) - zp[r]) * s[r]`` with two IEEE fp32
    roundings (:299), then cast to the runtime dtype (:300). Returns a uint16
    bf16 bit-pattern array (``out="bfloat16"``) or fp32 (``out="float32"``) of
    shape (out_dim, in_dim).
    """
    q = np.asarray(qweight)
    q2d = q.reshape(q.shape[0], -1)[:out_dim, :in_dim].astype(np.float32)
    s = np.asarray(scale).reshape(-1).astype(np.float32)[:out_dim]
    if zero_point is None:
        z = np.zeros(out_dim, dtype=np.float32)
    else:
        z = np.asarray(zero_point).reshape(-1).astype(np.float32)[:out_dim]
    v = (q2d - z[:, None]).astype(np.float32) * s[:, None]
    v = v.astype(np.float32)
    if out == "bfloat16":
        return bf16_rne_bits(v)
    if out == "float32":
        return v
    raise ValueError(f"unsupported output dtype {out!r}")


def cast_f32_bf16(x: np.ndarray) -> np.ndarray:
    """``param.to(torch.bfloat16)`` of src/stagehand/scheduler.py:181 / :1071 as bit patterns."""
    return bf16_rne_bits(np.asarray(x, dtype=np.float32).reshape(-1))


@dataclass(frozen=True)
class LayoutEntry:
    name: str
    shape: tuple[int, ...]
    dtype: str
    offset: int
    numel: int

    @property
    def nbytes(self) -> int:
        return self.numel * ITEMSIZE[self.dtype]


def build_param_layout(named_shapes: Sequence[tuple[str, Sequence[int]]], dtype: str) -> list[LayoutEntry]:
    """``_build_param_layout``, src/stagehand/scheduler.py:148-165.

    Parameters in ``named_parameters()`` order; offset is the running sum of
    numel * itemsize of the runtime dtype; no alignment padding.
    """
    out: list[LayoutEntry] = []
    off = 0
    for name, shape in named_shapes:
        numel = int(np.prod(shape, dtype=np.int64)) if len(shape) else 1
        out.append(LayoutEntry(name, tuple(int(s) for s in shape), dtype, off, numel))
        off += numel * ITEMSIZE[dtype]
    return out


def _as_runtime_bytes(values: np.ndarray, dtype: str) -> bytes:
    v = np.asarray(values)
    if dtype == "bfloat16":
        if v.dtype == np.uint16:
            return v.reshape(-1).tobytes()
        return cast_f32_bf16(v.astype(np.float32)).tobytes()
    if dtype == "float32":
        return v.astype(np.float32).reshape(-1).tobytes()
    raise ValueError(f"unsupported runtime dtype {dtype!r}")


def flatten_params(params: Mapping[str, np.ndarray], layout: Sequence[LayoutEntry]) -> bytearray:
    """``_flatten_params_into_buffer``, src/stagehand/scheduler.py:168-181
    (also the per-param copy loop of ``_load_module_backed_direct``, :1064-1071):
    each param cast to the runtime dtype at its layout offset."""
    total = max((e.offset + e.nbytes for e in layout), default=0)
    buf = bytearray(total)
    for e in layout:
        buf[e.offset:e.offset + e.nbytes] = _as_runtime_bytes(params[e.name], e.dtype)
    return buf


@dataclass(frozen=True)
class SquareQSpec:
    """Mirror of ``SquareQParamSpec`` (src/stagehand/registry.py:54-63)."""

    param_name: str
    layer_name: str
    kind: str  # "weight" | "bias"
    out_features: int
    in_features: int
    padded_in_features: int


def stage_squareq_block(
    layout: Sequence[LayoutEntry],
    specs: Mapping[str, SquareQSpec],
    module_param_names: set[str],
    module_params: Mapping[str, np.ndarray | None],
    layers: Mapping[str, Any],
    module_param_cache: dict[str, np.ndarray] | None = None,
) -> bytearray:
    """``_copy_squareq_backed_params_into_buffer``, src/stagehand/scheduler.py:243-325.

    ``layers`` maps layer name → dict with optional ``qweight`` (int8),
    ``scale``/``zero_point`` (fp32), ``bias`` (fp32) numpy arrays.
    ``module_params`` maps param name → current data, ``None`` or a size-0
    array when the param was evicted (:313-322).
    Branch structure, in order:
      weight spec with qweight/scale/zero_point present: 0-d shape → zeros
        (:276-278); out<=0 or in<=0 → zeros (:281-283); scale/zp vectors
        shorter than out → zeros (:293-297); else dequant (:299-300);
      weight spec with any of the three missing → falls through to the module
        branch (:272-275 lead to :310);
      bias spec: bias present → cast (:304-306) else zeros (:307-308);
      spec whose layer is missing / not a dict → module branch (:267);
      module branch: live param of matching numel → cast, cache a copy
        (:310-318); evicted → cached copy (:319-322); else zeros (:325).
    """
    total = max((e.offset + e.nbytes for e in layout), default=0)
    buf = bytearray(total)

    def put(e: LayoutEntry, data: bytes) -> None:
        assert len(data) == e.nbytes, (e.name, len(data), e.nbytes)
        buf[e.offset:e.offset + e.nbytes] = data

    for e in layout:
        zero = bytes(e.nbytes)
        spec = specs.get(e.name)
        if spec is not None:
            layer = layers.get(spec.layer_name)
            if isinstance(layer, dict):
                if spec.kind == "weight":
                    q, s, z = layer.get("qweight"), layer.get("scale"), layer.get("zero_point")
                    if q is not None and s is not None and z is not None:
                        if len(e.shape) == 0:
                            put(e, zero)
                            continue
                        out_dim = int(e.shape[0])
                        in_flat = int(e.numel // max(out_dim, 1))
                        if out_dim <= 0 or in_flat <= 0:
                            put(e, zero)
                            continue
                        sv = np.asarray(s).reshape(-1)
                        zv = np.asarray(z).reshape(-1)
                        if sv[:out_dim].size != out_dim or zv[:out_dim].size != out_dim:
                            put(e, zero)
                            continue
                        w = dequant_rows(q, sv, zv, out_dim, in_flat, out="float32")
                        put(e, _as_runtime_bytes(w, e.dtype))
                        continue
                elif spec.kind == "bias":
                    b = layer.get("bias")
                    if b is not None:
                        put(e, _as_runtime_bytes(np.asarray(b, dtype=np.float32), e.dtype))
                        continue
                    put(e, zero)
                    continue

        if e.name in module_param_names and e.name in module_params:
            p = module_params[e.name]
            if p is not None and np.asarray(p).size == e.numel:
                put(e, _as_runtime_bytes(np.asarray(p), e.dtype))
                if module_param_cache is not None and e.name not in module_param_cache:
                    module_param_cache[e.name] = np.array(p, copy=True)
                continue
            if module_param_cache is not None and e.name in module_param_cache:
                put(e, _as_runtime_bytes(module_param_cache[e.name], e.dtype))
                continue
        put(e, zero)
    return buf
