"""Block registry: model topology → ordered swappable blocks, and the
conversion of block parameters to file-backed / SquareQ-backed sources.

Semantics follow src/stagehand/registry.py (block discovery :391-439,
validation :441-455, safetensors headers :175-238, key aliasing :240-337,
SquareQ manifests :339-387 / :823-847, conversions :457-978, layer-mode
registration :1010-1046). The four conversions share one implementation here:
each walks a block's ``named_parameters()``, builds the runtime layout
(offset = running sum of numel * itemsize, no padding), keeps trainable,
normalisation and unmatched parameters module-backed, and records a source
spec for the rest.
"""
from __future__ import annotations

import json
import re
import struct
import weakref
from collections import OrderedDict
from dataclasses import dataclass, field, replace
from pathlib import Path
from typing import Callable

import torch
from torch import nn

from stagehand_amd.errors import StagehandOOMError

__all__ = ["BlockEntry", "BlockRegistry", "FileParamSpec", "SquareQParamSpec", "ParamLayoutEntry"]

ParamLayoutEntry = tuple[str, tuple[int, ...], torch.dtype, int, int]

_SAFETENSORS_DTYPES: dict[str, torch.dtype] = {
    "F16": torch.float16,
    "BF16": torch.bfloat16,
    "F32": torch.float32,
    "F64": torch.float64,
    "I8": torch.int8,
    "I16": torch.int16,
    "I32": torch.int32,
    "I64": torch.int64,
    "U8": torch.uint8,
}

# Adapter wrappers that rename a base parameter (``to_q.orig.weight``) while the
# checkpoint keeps the original key, and known checkpoint/diffusers name pairs;
# the table is the reference's (src/stagehand/registry.py:254-280) so that the
# same checkpoints resolve to the same tensors.
_WRAPPER_TOKENS = (".orig.", ".org_module.", ".base_layer.")
_NAME_ALIASES = (
    ("attn1.", "self_attn."), ("attn2.", "cross_attn."), ("to_q.", "q."), ("to_k.", "k."), ("to_v.", "v."),
    ("to_out.0.", "o."), ("ffn.net.0.proj.", "ffn.0."), ("ffn.net.2.", "ffn.2."), ("norm2.", "norm3."),
    (".attn1.", ".self_attn."), (".attn2.", ".cross_attn."), (".to_q.", ".q."), (".to_k.", ".k."),
    (".to_v.", ".v."), (".to_out.0.", ".o."), (".ffn.net.0.proj.", ".ffn.0."), (".ffn.net.2.", ".ffn.2."),
    (".norm2.", ".norm3."), ("scale_shift_table", "modulation"),
    ("ff.net.0.proj", "ff.linear_in"), ("ff.net.2", "ff.linear_out"),
    ("ff_context.net.0.proj", "ff_context.linear_in"), ("ff_context.net.2", "ff_context.linear_out"),
)
_KEY_PREFIXES = ("", "model.diffusion_model.", "diffusion_model.", "model.")
_NORM_TYPES = (nn.RMSNorm, nn.LayerNorm, nn.GroupNorm, nn.BatchNorm1d, nn.BatchNorm2d, nn.BatchNorm3d)


@dataclass(frozen=True)
class FileParamSpec:
    """A parameter read from a safetensors file (src/stagehand/registry.py:42-51)."""

    param_name: str
    file_offset: int
    source_nbytes: int
    source_dtype: torch.dtype
    source_shape: tuple[int, ...]
    file_path: str = ""


@dataclass(frozen=True)
class SquareQParamSpec:
    """A parameter read from a SquareQ INT8 slab (src/stagehand/registry.py:54-63)."""

    param_name: str
    layer_name: str
    kind: str  # "weight" | "bias"
    out_features: int
    in_features: int
    padded_in_features: int


def _param_size_bytes(module: nn.Module, dtype: torch.dtype) -> int:
    return sum(p.numel() for p in module.parameters()) * dtype.itemsize


def _resolve_param_owner(module: nn.Module, dotted_name: str) -> tuple[nn.Module | None, str | None]:
    parts = dotted_name.split(".")
    owner: nn.Module | None = module
    for part in parts[:-1]:
        if owner is None or not hasattr(owner, part):
            return None, None
        owner = getattr(owner, part)
    return owner, (parts[-1] if parts else None)


def _should_keep_module_param_resident(module: nn.Module, dotted_name: str, param: nn.Parameter) -> bool:
    """Normalisation weights/biases stay module-backed (src/stagehand/registry.py:88-111)."""
    owner, leaf = _resolve_param_owner(module, dotted_name)
    if owner is None or leaf not in {"weight", "bias"}:
        return False
    if isinstance(owner, _NORM_TYPES):
        return True
    return "norm" in owner.__class__.__name__.lower() and int(param.ndim) <= 1


@dataclass(frozen=True)
class BlockEntry:
    """Immutable descriptor of one swappable block (src/stagehand/registry.py:117-155)."""

    block_id: str
    module_ref: weakref.ref
    size_bytes: int
    dtype: torch.dtype
    dependencies: tuple[str, ...]
    group: str
    exec_order: int
    quant_format: str | None = None
    quant_meta_bytes: int = 0
    eriquant_qtype: str | None = None
    source_path: str | None = None
    source_format: str | None = None
    param_layout: tuple[ParamLayoutEntry, ...] = field(default_factory=tuple)
    file_param_specs: tuple[FileParamSpec, ...] = field(default_factory=tuple)
    squareq_param_specs: tuple[SquareQParamSpec, ...] = field(default_factory=tuple)
    module_param_names: tuple[str, ...] = field(default_factory=tuple)

    @property
    def file_backed(self) -> bool:
        return self.source_path is not None and (len(self.file_param_specs) > 0 or len(self.squareq_param_specs) > 0)

    @property
    def squareq_backed(self) -> bool:
        return self.source_format in ("squareq_bp8", "squareq_v2") and len(self.squareq_param_specs) > 0

    @property
    def eriquant_backed(self) -> bool:
        return self.quant_format == "eriquant"


def parse_safetensors_index(path: Path) -> dict[str, tuple[int, int, torch.dtype, tuple[int, ...]]]:
    """key → (absolute byte offset, nbytes, dtype, shape) from a safetensors header.

    Format: 8-byte little-endian header length, JSON header, data; a tensor's
    bytes start at 8 + header_len + data_offsets[0].
    """
    with Path(path).open("rb") as fh:
        raw = fh.read(8)
        if len(raw) != 8:
            raise ValueError(f"Invalid safetensors header for {path}")
        (hlen,) = struct.unpack("<Q", raw)
        header_bytes = fh.read(hlen)
        if len(header_bytes) != hlen:
            raise ValueError(f"Truncated safetensors header for {path}")
    header = json.loads(header_bytes.decode("utf-8"))
    base = 8 + hlen
    index: dict[str, tuple[int, int, torch.dtype, tuple[int, ...]]] = {}
    for key, meta in header.items():
        if key == "__metadata__" or not isinstance(meta, dict):
            continue
        offs, shape, dtype_name = meta.get("data_offsets"), meta.get("shape"), meta.get("dtype")
        if not (isinstance(offs, list) and len(offs) == 2 and isinstance(shape, list) and isinstance(dtype_name, str)):
            continue
        start, end = int(offs[0]), int(offs[1])
        if end < start:
            raise ValueError(f"Invalid data_offsets for key {key!r} in {path}")
        if dtype_name not in _SAFETENSORS_DTYPES:
            raise ValueError(f"Unsupported safetensors dtype {dtype_name!r}")
        index[key] = (base + start, end - start, _SAFETENSORS_DTYPES[dtype_name], tuple(int(d) for d in shape))
    return index


def candidate_tensor_keys(block_id: str, param_name: str) -> tuple[str, ...]:
    """Checkpoint keys a block parameter may be stored under, most direct first.

    Breadth-first over wrapper-token removals and name aliases, then every
    known key prefix (src/stagehand/registry.py:240-317).
    """
    names: list[str] = []
    seen: set[str] = set()
    frontier = [param_name]
    while frontier:
        cur = frontier.pop(0)
        if cur in seen:
            continue
        seen.add(cur)
        names.append(cur)
        variants = [cur.replace(tok, ".") for tok in _WRAPPER_TOKENS if tok in cur]
        variants += [cur.replace(a, b) for a, b in _NAME_ALIASES if a in cur]
        for v in variants:
            v = v.replace("..", ".").strip(".")
            if v and v not in seen:
                frontier.append(v)
    out: list[str] = []
    for prefix in _KEY_PREFIXES:
        for name in names:
            key = f"{prefix}{block_id}.{name}"
            if key not in out:
                out.append(key)
    return tuple(out)


def candidate_squareq_layer_keys(block_id: str, param_name: str) -> tuple[str, ...]:
    """SquareQ layer names a ``*.weight`` / ``*.bias`` parameter may belong to."""
    base = param_name
    if base.endswith(".weight"):
        base = base[: -len(".weight")]
    elif base.endswith(".bias"):
        base = base[: -len(".bias")]
    elif base in {"weight", "bias"}:
        base = ""
    for suffix in (".orig", ".org_module", ".base_layer"):
        if base.endswith(suffix):
            base = base[: -len(suffix)]
            break
    if not base:
        return (block_id,)
    return candidate_tensor_keys(block_id, base)


def load_squareq_v1_manifest(path: Path) -> dict[str, tuple[int, int, int, bool]]:
    """layer → (out, in, padded_in, has_bias) from a v1 ``.fpk``/``.slab`` torch.save payload."""
    payload = torch.load(str(path), map_location="cpu", weights_only=True, mmap=True)
    if not isinstance(payload, dict):
        raise ValueError(f"Invalid SquareQ slab payload in {path}")
    manifest = payload.get("manifest")
    if not isinstance(manifest, dict):
        raise ValueError(f"SquareQ slab missing manifest in {path}")
    layers = manifest.get("layers")
    if not isinstance(layers, list):
        raise ValueError(f"SquareQ manifest missing layers list in {path}")
    out: dict[str, tuple[int, int, int, bool]] = {}
    for layer in layers:
        if not isinstance(layer, dict):
            continue
        name = layer.get("name")
        if not isinstance(name, str) or not name:
            continue
        o, i = int(layer.get("out", 0)), int(layer.get("inp", 0))
        if o <= 0 or i <= 0:
            continue
        out[name] = (o, i, int(layer.get("padded_in", i)), bool(layer.get("has_bias", False)))
    return out


def load_squareq_v2_manifest(path: Path) -> dict[str, tuple[int, int, int, bool]]:
    """canonical_name → (out, in, padded_in, has_bias) from a v2 JSON manifest
    (fields canonical_name, orig_shape, packed_shape, bias_key)."""
    raw = json.loads(Path(path).read_text())
    out: dict[str, tuple[int, int, int, bool]] = {}
    for layer in raw.get("layers", []):
        name = layer.get("canonical_name", "")
        if not name:
            continue
        orig = layer.get("orig_shape", [0, 0])
        packed = layer.get("packed_shape", [0, 0])
        o = int(orig[0]) if len(orig) > 0 else 0
        i = int(orig[1]) if len(orig) > 1 else 0
        if o <= 0 or i <= 0:
            continue
        out[name] = (o, i, int(packed[1]) if len(packed) > 1 else i, layer.get("bias_key") is not None)
    return out


# A matcher decides, for one frozen non-norm parameter, which source spec (if
# any) backs it: returns a spec or None (→ module-backed).
_Matcher = Callable[[str, str, tuple[int, ...], int], object]


class BlockRegistry:
    """Ordered registry of swappable blocks; frozen by ``validate``."""

    def __init__(self) -> None:
        self._entries: OrderedDict[str, BlockEntry] = OrderedDict()
        self._frozen = False

    # kept as static methods for callers of the reference's private helpers
    _parse_safetensors_index = staticmethod(parse_safetensors_index)
    _candidate_tensor_keys = staticmethod(candidate_tensor_keys)
    _candidate_squareq_layer_keys = staticmethod(candidate_squareq_layer_keys)
    _load_squareq_manifest = staticmethod(load_squareq_v1_manifest)
    _load_v2_manifest = staticmethod(load_squareq_v2_manifest)

    @staticmethod
    def _decode_safetensors_dtype(dtype_name: str) -> torch.dtype:
        if dtype_name not in _SAFETENSORS_DTYPES:
            raise ValueError(f"Unsupported safetensors dtype {dtype_name!r}")
        return _SAFETENSORS_DTYPES[dtype_name]

    # ── construction ─────────────────────────────────────────────────

    def build_from_model(self, model: nn.Module, block_pattern: str, group: str, dtype: torch.dtype) -> None:
        if self._frozen:
            raise RuntimeError("Cannot build_from_model on a frozen registry")
        rx = re.compile(block_pattern)
        order = len(self._entries)
        for name, module in model.named_modules():
            if name and rx.search(name):
                self._entries[name] = BlockEntry(name, weakref.ref(module), _param_size_bytes(module, dtype), dtype,
                                                 (), group, order)
                order += 1

    def build_from_module_list(self, modules: list[tuple[str, nn.Module]], group: str, dtype: torch.dtype) -> None:
        if self._frozen:
            raise RuntimeError("Cannot build_from_module_list on a frozen registry")
        seen: set[int] = set()
        order = len(self._entries)
        for name, module in modules:
            if id(module) in seen:
                continue
            seen.add(id(module))
            self._entries[name] = BlockEntry(name, weakref.ref(module), _param_size_bytes(module, dtype), dtype,
                                             (), group, order)
            order += 1

    def validate(self, pool_capacity_bytes: int) -> None:
        for entry in self._entries.values():
            if entry.size_bytes > pool_capacity_bytes:
                raise StagehandOOMError(
                    f"Block {entry.block_id!r} ({entry.size_bytes} bytes) exceeds pool capacity ({pool_capacity_bytes} bytes)"
                )
        self._frozen = True

    @property
    def frozen(self) -> bool:
        return self._frozen

    # ── source conversion ────────────────────────────────────────────

    def _convert(self, matcher: _Matcher, source_path: str, source_format: str, kind: str,
                 drop_module_tensors: bool) -> int:
        converted = 0
        new_entries: OrderedDict[str, BlockEntry] = OrderedDict()
        for block_id, entry in self._entries.items():
            module = entry.module_ref()
            if module is None:
                new_entries[block_id] = entry
                continue
            layout: list[ParamLayoutEntry] = []
            specs: list = []
            module_names: list[str] = []
            offset = 0
            for pname, param in module.named_parameters():
                shape = tuple(int(d) for d in param.shape)
                numel = int(param.numel())
                layout.append((pname, shape, entry.dtype, offset, numel))
                offset += numel * entry.dtype.itemsize
                spec = None
                if not param.requires_grad and not _should_keep_module_param_resident(module, pname, param):
                    spec = matcher(block_id, pname, shape, numel)
                if spec is None:
                    module_names.append(pname)
                    continue
                specs.append(spec)
                converted += 1
                if drop_module_tensors:
                    with torch.no_grad():
                        param.data = torch.empty(0, dtype=param.dtype, device=param.device)
                        param.grad = None
            if specs:
                new_entries[block_id] = replace(
                    entry,
                    source_path=source_path,
                    source_format=source_format,
                    param_layout=tuple(layout),
                    file_param_specs=tuple(specs) if kind == "file" else tuple(),
                    squareq_param_specs=tuple(specs) if kind == "squareq" else tuple(),
                    module_param_names=tuple(module_names),
                )
            else:
                new_entries[block_id] = entry
        self._entries = new_entries
        return converted

    @staticmethod
    def _file_matcher(index: dict) -> _Matcher:
        def match(block_id: str, pname: str, shape: tuple[int, ...], numel: int):
            for key in candidate_tensor_keys(block_id, pname):
                meta = index.get(key)
                if meta is None:
                    continue
                off, nbytes, dt, src_shape = meta[:4]
                if src_shape != shape:
                    return None
                return FileParamSpec(pname, off, nbytes, dt, src_shape, meta[4] if len(meta) > 4 else "")
            return None
        return match

    @staticmethod
    def _squareq_matcher(layer_meta: dict[str, tuple[int, int, int, bool]]) -> _Matcher:
        def match(block_id: str, pname: str, shape: tuple[int, ...], numel: int):
            if pname.endswith(".weight") or pname == "weight":
                kind = "weight"
            elif pname.endswith(".bias") or pname == "bias":
                kind = "bias"
            else:
                return None
            for layer in candidate_squareq_layer_keys(block_id, pname):
                meta = layer_meta.get(layer)
                if meta is None:
                    continue
                out_f, in_f, padded_in, has_bias = meta
                if kind == "weight":
                    if len(shape) == 0:
                        return None
                    out_dim = int(shape[0])
                    in_flat = numel // max(out_dim, 1)
                    if out_dim != out_f or in_flat != in_f or out_dim <= 0 or in_flat <= 0:
                        return None
                elif not has_bias or numel != out_f:
                    return None
                return SquareQParamSpec(pname, layer, kind, out_f, in_f, padded_in)
            return None
        return match

    def _require_frozen(self, what: str) -> None:
        if not self._frozen:
            raise RuntimeError(f"{what} requires a validated (frozen) registry")

    def convert_to_file_backed(self, source_path: str | Path, *, drop_module_tensors: bool = True) -> int:
        self._require_frozen("convert_to_file_backed")
        path = Path(source_path).expanduser()
        if not path.exists():
            raise FileNotFoundError(f"file-backed source not found: {path}")
        if path.suffix.lower() in {".fpk", ".slab"}:
            return self.convert_to_squareq_backed(path, drop_module_tensors=drop_module_tensors)
        index = parse_safetensors_index(path)
        return self._convert(self._file_matcher(index), str(path), "safetensors", "file", drop_module_tensors)

    def convert_to_file_backed_sharded(self, source_dir: str | Path, *, drop_module_tensors: bool = True) -> int:
        self._require_frozen("convert_to_file_backed_sharded")
        d = Path(source_dir).expanduser()
        if not d.is_dir():
            raise FileNotFoundError(f"Sharded source directory not found: {d}")
        idx_path = d / "diffusion_pytorch_model.safetensors.index.json"
        if not idx_path.exists():
            idx_path = d / "model.safetensors.index.json"
        if not idx_path.exists():
            raise FileNotFoundError(f"No safetensors index found in {d}. Expected diffusion_pytorch_model.safetensors.index.json")
        weight_map: dict[str, str] = json.loads(idx_path.read_text()).get("weight_map", {})
        if not weight_map:
            raise ValueError(f"Empty weight_map in {idx_path}")
        unified: dict[str, tuple] = {}
        for shard in dict.fromkeys(weight_map.values()):
            shard_path = d / shard
            if not shard_path.exists():
                raise FileNotFoundError(f"Shard file not found: {shard_path}")
            for key, meta in parse_safetensors_index(shard_path).items():
                unified[key] = (*meta, str(shard_path))
        return self._convert(self._file_matcher(unified), str(d), "safetensors_sharded", "file", drop_module_tensors)

    def convert_to_squareq_backed(self, squareq_path: str | Path, *, drop_module_tensors: bool = True) -> int:
        self._require_frozen("convert_to_squareq_backed")
        path = Path(squareq_path).expanduser()
        if not path.exists():
            raise FileNotFoundError(f"SquareQ slab file not found: {path}")
        meta = load_squareq_v1_manifest(path)
        return self._convert(self._squareq_matcher(meta), str(path), "squareq_bp8", "squareq", drop_module_tensors)

    def convert_to_squareq_v2_backed(self, safetensors_path: str | Path, manifest_path: str | Path, *,
                                     drop_module_tensors: bool = True) -> int:
        self._require_frozen("convert_to_squareq_v2_backed")
        st_path = Path(safetensors_path).expanduser()
        mf_path = Path(manifest_path).expanduser()
        if not st_path.exists():
            raise FileNotFoundError(f"V2 safetensors file not found: {st_path}")
        if not mf_path.exists():
            raise FileNotFoundError(f"V2 manifest file not found: {mf_path}")
        meta = load_squareq_v2_manifest(mf_path)
        return self._convert(self._squareq_matcher(meta), str(st_path), "squareq_v2", "squareq", drop_module_tensors)

    def mark_eriquant_backed(self, block_ids: list[str], qtype_name: str, frozen_sizes: dict[str, int] | None = None) -> None:
        for bid in block_ids:
            if bid not in self._entries:
                continue
            kw: dict[str, object] = {"quant_format": "eriquant", "eriquant_qtype": qtype_name}
            if frozen_sizes is not None and bid in frozen_sizes:
                kw["size_bytes"] = frozen_sizes[bid]
            self._entries[bid] = replace(self._entries[bid], **kw)

    # ── queries ──────────────────────────────────────────────────────

    def get(self, block_id: str) -> BlockEntry:
        return self._entries[block_id]

    def blocks_in_order(self) -> list[BlockEntry]:
        return sorted(self._entries.values(), key=lambda e: e.exec_order)

    def __len__(self) -> int:
        return len(self._entries)

    def groups(self) -> dict[str, list[BlockEntry]]:
        out: dict[str, list[BlockEntry]] = {}
        for e in self._entries.values():
            out.setdefault(e.group, []).append(e)
        return out

    def __contains__(self, block_id: str) -> bool:
        return block_id in self._entries

    def __repr__(self) -> str:
        return f"BlockRegistry(blocks={len(self)}, frozen={self._frozen})"
