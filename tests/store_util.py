"""Writes MLX-style safetensors model directories for the weight-store tests.

A safetensors file is an 8-byte little-endian header length, a JSON header
{name: {dtype, shape, data_offsets}} and the raw tensor bytes; the directory's
model.safetensors.index.json maps each tensor to its shard.
"""
from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np

DTYPES = {np.dtype(np.uint32): "U32", np.dtype(np.uint16): "BF16", np.dtype(np.float32): "F32",
          np.dtype(np.int8): "I8"}


def write_shard(path: Path, tensors: dict, header_override: dict | None = None, pad_header: int = 0) -> None:
    """tensors: name -> numpy array (uint16 is written as BF16)."""
    header, blobs, off = {}, [], 0
    for name, arr in tensors.items():
        arr = np.ascontiguousarray(arr)
        raw = arr.tobytes()
        header[name] = {"dtype": DTYPES[arr.dtype], "shape": list(arr.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    header["__metadata__"] = {"format": "mlx"}
    if header_override:
        header.update(header_override)
    text = json.dumps(header).encode() + b" " * pad_header
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)))
        f.write(text)
        for b in blobs:
            f.write(b)


def write_model(root: Path, shards: dict, index_extra: dict | None = None) -> Path:
    """shards: file name -> {tensor name: array}."""
    root.mkdir(parents=True, exist_ok=True)
    weight_map = {}
    for fname, tensors in shards.items():
        write_shard(root / fname, tensors)
        for name in tensors:
            weight_map[name] = fname
    if index_extra:
        weight_map.update(index_extra)
    (root / "model.safetensors.index.json").write_text(
        json.dumps({"metadata": {"total_size": 0}, "weight_map": weight_map}))
    return root


def q4_tensors(base: str, packed, scales, biases) -> dict:
    return {f"{base}.weight": packed, f"{base}.scales": scales, f"{base}.biases": biases}
