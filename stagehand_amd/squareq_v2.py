"""Reader of SquareQ V2 slabs: a safetensors file + ``<stem>.manifest.json``.

The reference registers V2 layers from the manifest fields ``canonical_name``,
``orig_shape``, ``packed_shape`` and ``bias_key`` (src/stagehand/registry.py:823-847)
and loads the layer tensors through an external package
(src/stagehand/scheduler.py:631-649) that is not part of the reference. The
tensor naming used here is therefore this build's: a manifest layer may name
its tensors with ``qweight_key``, ``scale_key``, ``zero_point_key`` and
``bias_key``; otherwise they are ``<canonical_name>.qweight`` / ``.scale`` /
``.zero_point``, and a missing zero point means zeros. Tensors are zero-copy
views of the memory-mapped file, so the loader's host copy reads the mapped
pages directly into the pinned slab.
"""
from __future__ import annotations

import json
import warnings
from pathlib import Path
from typing import Any

import torch

from stagehand_amd.registry import parse_safetensors_index

__all__ = ["read_v2_layers", "write_v2_slab"]


def read_v2_layers(safetensors_path: str, manifest_path: str, file_view: memoryview) -> dict[str, dict[str, Any]]:
    index = parse_safetensors_index(Path(safetensors_path))
    manifest = json.loads(Path(manifest_path).read_text())

    def tensor(key: str | None) -> torch.Tensor | None:
        if not key or key not in index:
            return None
        off, nbytes, dtype, shape = index[key]
        with warnings.catch_warnings():
            warnings.simplefilter("ignore", UserWarning)
            return torch.frombuffer(file_view[off:off + nbytes], dtype=dtype).reshape(shape)

    layers: dict[str, dict[str, Any]] = {}
    for entry in manifest.get("layers", []):
        name = entry.get("canonical_name", "")
        if not name:
            continue
        q = tensor(entry.get("qweight_key", f"{name}.qweight"))
        s = tensor(entry.get("scale_key", f"{name}.scale"))
        z = tensor(entry.get("zero_point_key", f"{name}.zero_point"))
        if z is None and s is not None:
            z = torch.zeros(s.numel(), dtype=torch.float32)
        layer: dict[str, Any] = {"qweight": q, "scale": s, "zero_point": z}
        b = tensor(entry.get("bias_key"))
        if b is not None:
            layer["bias"] = b
        layers[name] = layer
    return layers


def write_v2_slab(path: str, layers: dict[str, dict[str, torch.Tensor]]) -> str:
    """Writes ``path`` (safetensors) and its manifest from layer → {qweight, scale, [zero_point], [bias]}."""
    from safetensors.torch import save_file

    tensors: dict[str, torch.Tensor] = {}
    entries = []
    for name, t in layers.items():
        q = t["qweight"]
        tensors[f"{name}.qweight"] = q.contiguous()
        tensors[f"{name}.scale"] = t["scale"].contiguous()
        e = {"canonical_name": name, "orig_shape": [int(q.shape[0]), int(t.get("in_features", q.shape[1]))],
             "packed_shape": [int(q.shape[0]), int(q.shape[1])], "bias_key": None}
        if "zero_point" in t:
            tensors[f"{name}.zero_point"] = t["zero_point"].contiguous()
        if "bias" in t:
            tensors[f"{name}.bias"] = t["bias"].contiguous()
            e["bias_key"] = f"{name}.bias"
        entries.append(e)
    save_file(tensors, path)
    manifest = str(Path(path).with_suffix(".manifest.json"))
    Path(manifest).write_text(json.dumps({"format": "squareq_v2", "layers": entries}))
    return manifest
