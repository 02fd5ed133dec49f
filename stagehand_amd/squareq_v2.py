"""Reader of SquareQ V2 slabs: a safetensors file + ``<stem>.manifest.json``.

The reference registers V2 layers from the manifest fields ``canonical_name``,
``orig_shape``, ``packed_shape`` and ``bias_key`` (src/stagehand/registry.py:823-847)
and loads the layer tensors through an external package
(src/stagehand/scheduler.py:631-649) that is not part of the reference. The
tensor naming used here is therefore this build's: a manifest layer may name
its tensors with ``qweight_key``, ``scale_key``, ``zero_point_key`` and
``bias_key``; otherwise they are ``<canonical_name>.qweight`` / ``.scale`` /
``.zero_point``, and a missing zero point means zeros. ``read_v2_layers``
gives zero-copy views of the memory-mapped file (the loader's host copy reads
the mapped pages into the pinned slab); ``read_v2_locations`` gives each
tensor's byte range in the file instead, for the native weight-file reader,
which reads the int8 rows and scales straight into the slab.
"""
from __future__ import annotations

import json
import warnings
from pathlib import Path
from typing import Any

import torch

from stagehand_amd.registry import parse_safetensors_index

__all__ = ["read_v2_layers", "read_v2_locations", "write_v2_slab"]

# (file offset, bytes, dtype, shape) of one tensor
Location = tuple[int, int, torch.dtype, tuple[int, ...]]


def read_v2_locations(safetensors_path: str, manifest_path: str) -> dict[str, dict[str, Location]]:
    """layer → {"qweight", "scale", ["zero_point"], ["bias"]} → where the tensor lies in the file."""
    index = parse_safetensors_index(Path(safetensors_path))
    manifest = json.loads(Path(manifest_path).read_text())
    layers: dict[str, dict[str, Location]] = {}
    for entry in manifest.get("layers", []):
        name = entry.get("canonical_name", "")
        if not name:
            continue
        keys = {"qweight": entry.get("qweight_key", f"{name}.qweight"),
                "scale": entry.get("scale_key", f"{name}.scale"),
                "zero_point": entry.get("zero_point_key", f"{name}.zero_point"),
                "bias": entry.get("bias_key")}
        layers[name] = {what: tuple(index[k]) for what, k in keys.items() if k and k in index}
    return layers


def read_v2_layers(safetensors_path: str, manifest_path: str, file_view: memoryview) -> dict[str, dict[str, Any]]:
    """layer → {"qweight", "scale", "zero_point", ["bias"]} as views of the mapped file (a
    missing zero point is zeros), the layer dict of src/stagehand/scheduler.py:285-308."""
    layers: dict[str, dict[str, Any]] = {}
    for name, loc in read_v2_locations(safetensors_path, manifest_path).items():
        views: dict[str, Any] = {}
        for what, (off, nbytes, dtype, shape) in loc.items():
            with warnings.catch_warnings():
                warnings.simplefilter("ignore", UserWarning)
                views[what] = torch.frombuffer(file_view[off:off + nbytes], dtype=dtype).reshape(shape)
        s = views.get("scale")
        layer: dict[str, Any] = {"qweight": views.get("qweight"), "scale": s, "zero_point": views.get("zero_point")}
        if layer["zero_point"] is None and s is not None:
            layer["zero_point"] = torch.zeros(s.numel(), dtype=torch.float32)
        if "bias" in views:
            layer["bias"] = views["bias"]
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
