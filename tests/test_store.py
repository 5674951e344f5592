"""MLX safetensors weight store on the host (no GPU work): the index / shard /
header rules of open_mlx_safetensors_dir, read_safetensors_header,
validate_tensor_range and resolve_shard (/root/reference/src/model.rs:136-197,
312-431), through the C-ABI (qm_store_open / qm_store_tensor_info)."""
from __future__ import annotations

import json
import struct

import numpy as np
import pytest

from qm38 import QmError, WeightStore, load, synth
from store_util import q4_tensors, write_model, write_shard


def _q4(rng, rows, K):
    return synth.q4_matrix(rng, rows, K)


def test_multi_shard_index_and_tensor_info(tmp_path):
    rng = np.random.default_rng(1)
    a = q4_tensors("model.layers.0.mlp.gate_proj", *_q4(rng, 96, 256))
    b = q4_tensors("model.layers.0.mlp.up_proj", *_q4(rng, 40, 128))
    extra = {"model.norm.weight": np.arange(7, dtype=np.float32)}
    root = write_model(tmp_path / "m", {"model-00001-of-00002.safetensors": {**a, **extra},
                                        "model-00002-of-00002.safetensors": b})
    st = WeightStore(root)
    assert len(st) == 7
    assert st.info("model.layers.0.mlp.gate_proj.weight") == ("U32", (96, 32), 96 * 32 * 4)
    assert st.info("model.layers.0.mlp.gate_proj.scales") == ("BF16", (96, 4), 96 * 4 * 2)
    assert st.info("model.layers.0.mlp.up_proj.biases") == ("BF16", (40, 2), 40 * 2 * 2)
    assert st.info("model.norm.weight") == ("F32", (7,), 28)
    with pytest.raises(QmError, match="INVALID_TENSOR"):
        st.info("model.layers.1.mlp.gate_proj.weight")
    st.close()


def test_tensors_not_in_the_index_are_not_exposed(tmp_path):
    # Only indexed tensors are part of the store (the shard may hold more).
    root = tmp_path / "m"
    root.mkdir()
    write_shard(root / "s.safetensors", {"x": np.zeros(4, np.float32), "y": np.ones(2, np.float32)})
    (root / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {"x": "s.safetensors"}}))
    st = WeightStore(root)
    assert len(st) == 1 and st.info("x")[1] == (4,)
    with pytest.raises(QmError):
        st.info("y")


def test_unicode_and_escaped_names(tmp_path):
    name = 'model.layers.0.é\\"q'
    root = write_model(tmp_path / "m", {"s.safetensors": {name: np.zeros(3, np.float32)}})
    assert WeightStore(root).info(name) == ("F32", (3,), 12)


@pytest.mark.parametrize("shard", ["../outside.safetensors", "/abs/path.safetensors", "a/../b.safetensors",
                                   "./s.safetensors"])
def test_rejects_unsafe_shard_paths(tmp_path, shard):
    root = write_model(tmp_path / "m", {"s.safetensors": {"x": np.zeros(1, np.float32)}},
                       index_extra={"y": shard})
    with pytest.raises(QmError, match="MODEL_FORMAT"):
        WeightStore(root)


def test_missing_index_shard_and_indexed_tensor(tmp_path):
    with pytest.raises(QmError, match="MODEL_FORMAT"):
        WeightStore(tmp_path / "nothing")
    root = write_model(tmp_path / "a", {"s.safetensors": {"x": np.zeros(1, np.float32)}},
                       index_extra={"y": "missing.safetensors"})
    with pytest.raises(QmError, match="MODEL_FORMAT"):
        WeightStore(root)
    root = write_model(tmp_path / "b", {"s.safetensors": {"x": np.zeros(1, np.float32)}},
                       index_extra={"z": "s.safetensors"})
    with pytest.raises(QmError, match="MODEL_FORMAT"):
        WeightStore(root)


def test_rejects_bad_headers(tmp_path):
    def model_with(write):
        root = tmp_path / f"m{len(list(tmp_path.iterdir()))}"
        root.mkdir()
        write(root / "s.safetensors")
        (root / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {"x": "s.safetensors"}}))
        return root

    cases = [
        lambda p: p.write_bytes(b"\x01\x02"),                                     # shorter than the length field
        lambda p: p.write_bytes(struct.pack("<Q", 1 << 40) + b"{}"),              # header longer than the file
        lambda p: p.write_bytes(struct.pack("<Q", 2) + b"[]"),                    # not an object
        lambda p: p.write_bytes(struct.pack("<Q", 5) + b"{\"x\":"),               # truncated JSON
        lambda p: write_shard(p, {"x": np.zeros(2, np.float32)},                  # data past the end
                              header_override={"x": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}),
        lambda p: write_shard(p, {"x": np.zeros(2, np.float32)},                  # reversed offsets
                              header_override={"x": {"dtype": "F32", "shape": [2], "data_offsets": [8, 0]}}),
        lambda p: write_shard(p, {"x": np.zeros(2, np.float32)},                  # empty shape (scalar)
                              header_override={"x": {"dtype": "F32", "shape": [], "data_offsets": [0, 4]}}),
        lambda p: write_shard(p, {"x": np.zeros(2, np.float32)},                  # empty dtype
                              header_override={"x": {"dtype": "", "shape": [2], "data_offsets": [0, 8]}}),
        lambda p: write_shard(p, {"x": np.zeros(2, np.float32)},                  # negative offset
                              header_override={"x": {"dtype": "F32", "shape": [2], "data_offsets": [-1, 8]}}),
    ]
    for make in cases:
        with pytest.raises(QmError, match="MODEL_FORMAT"):
            WeightStore(model_with(make))


def test_header_padding_and_metadata_are_accepted(tmp_path):
    root = tmp_path / "m"
    root.mkdir()
    write_shard(root / "s.safetensors", {"x": np.arange(5, dtype=np.float32)}, pad_header=13)
    (root / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {"x": "s.safetensors"}}))
    assert WeightStore(root).info("x") == ("F32", (5,), 20)


def test_store_symbols_exported():
    lib = load()
    for n in ("qm_store_open", "qm_store_close", "qm_store_tensor_info", "qm_store_upload", "qm_store_upload_q4"):
        assert hasattr(lib, n)
