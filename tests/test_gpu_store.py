"""Q4 matrices uploaded from an MLX safetensors directory (qm_store_upload_q4;
Q4AffineMatrix::from_store / validate_affine_tensor, native.rs:5384-5516) run
the same projections as directly uploaded arrays: outputs bit-equal to the
direct path and within the oracle tolerance; malformed Q4 groups rejected
with the reference's error kinds."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from gpu_util import assert_bf16_close, bf16_dev_to_f32, empty_bf16, from_dev, to_dev
from qm38 import QmError, WeightStore, synth
from store_util import q4_tensors, write_model

pytestmark = pytest.mark.gpu


def test_store_q4_projection_matches_direct_upload(rt, torch_dev, tmp_path):
    import qm38
    rng = np.random.default_rng(3)
    K = 512
    mats = {"model.layers.0.self_attn.q_proj": synth.q4_matrix(rng, 320, K),
            "model.layers.0.self_attn.k_proj": synth.q4_matrix(rng, 64, K),
            "model.layers.0.mlp.down_proj": synth.q4_matrix(rng, 200, K)}
    names = list(mats)
    root = write_model(tmp_path / "m", {"a.safetensors": {**q4_tensors(names[0], *mats[names[0]]),
                                                          **q4_tensors(names[1], *mats[names[1]])},
                                        "b.safetensors": q4_tensors(names[2], *mats[names[2]])})
    st = WeightStore(root)
    jobs = [st.upload_q4(rt, n + ".weight") for n in names]
    assert [j.in_elems for j in jobs] == [K] * 3 and [j.out_rows for j in jobs] == [320, 64, 200]
    direct = [qm38.Runtime.job(to_dev(w, torch_dev), to_dev(s, torch_dev), to_dev(b, torch_dev), w.shape[0])
              for w, s, b in mats.values()]
    for M in (1, 4, 40):
        xb = synth.bf16_normal(rng, (M, K))
        x = to_dev(xb, torch_dev)
        outs_s = [empty_bf16((M, j.out_rows), torch_dev) for j in jobs]
        outs_d = [empty_bf16((M, j.out_rows), torch_dev) for j in jobs]
        rt.q4_project(jobs, x, K, M, outs_s)
        rt.q4_project(direct, x, K, M, outs_d)
        for (w, s, b), o_s, o_d in zip(mats.values(), outs_s, outs_d):
            np.testing.assert_array_equal(from_dev(o_s), from_dev(o_d))
            assert_bf16_close(bf16_dev_to_f32(o_s), oracle.q4_project(xb, w, s, b), what=f"store M{M}")
    # raw bytes of any tensor
    buf = st.upload(rt, names[0] + ".scales")
    assert buf.nbytes == mats[names[0]][1].nbytes
    import torch
    host = np.empty(mats[names[0]][1].shape, np.uint16)
    torch.cuda.synchronize()
    rt.lib.qm_copy_to_host(rt.handle, host.ctypes.data, buf.data_ptr(), host.nbytes)
    np.testing.assert_array_equal(host, mats[names[0]][1])
    st.close()


def test_store_rejects_malformed_q4_groups(rt, torch_dev, tmp_path):
    rng = np.random.default_rng(4)
    w, s, b = synth.q4_matrix(rng, 16, 128)
    cases = {
        "wrong_weight_dtype": {"x.weight": w.view(np.float32), "x.scales": s, "x.biases": b},
        "scales_shape": {"x.weight": w, "x.scales": s[:, :1].copy(), "x.biases": b},
        "biases_dtype": {"x.weight": w, "x.scales": s, "x.biases": b.astype(np.float32)},
        "missing_biases": {"x.weight": w, "x.scales": s},
        "ungrouped_k": {"x.weight": w[:, :4].copy(), "x.scales": s[:, :1].copy(), "x.biases": b[:, :1].copy()},
        "weight_vector": {"x.weight": w[0].copy(), "x.scales": s, "x.biases": b},
    }
    for i, (label, tensors) in enumerate(cases.items()):
        st = WeightStore(write_model(tmp_path / f"c{i}", {"s.safetensors": tensors}))
        with pytest.raises(QmError, match="INVALID_TENSOR"):
            st.upload_q4(rt, "x.weight")
        st.close()
    st = WeightStore(write_model(tmp_path / "ok", {"s.safetensors": {"x.weight": w, "x.scales": s, "x.biases": b,
                                                                     "y": s}}))
    with pytest.raises(QmError, match="INVALID_TENSOR"):  # not a .weight name
        st.upload_q4(rt, "y")
    j = st.upload_q4(rt, "x.weight")
    assert (j.out_rows, j.in_elems) == (16, 128)


def test_reference_layout_cases(rt, torch_dev, tmp_path):
    # native.rs:5731 accepts_an_mlx_q4_affine_matrix_layout and :5745
    # rejects_a_wrong_scale_layout: U32 [3, 16] with BF16 [3, 2] scales and
    # biases is a 3 x 128 matrix; BF16 [3, 3] scales are rejected.
    w = np.arange(48, dtype=np.uint32).reshape(3, 16)
    s2 = np.full((3, 2), 0x3F80, np.uint16)
    s3 = np.full((3, 3), 0x3F80, np.uint16)
    ok = WeightStore(write_model(tmp_path / "ok", {"s.safetensors": {"layer.weight": w, "layer.scales": s2,
                                                                     "layer.biases": s2}}))
    j = ok.upload_q4(rt, "layer.weight")
    assert (j.out_rows, j.in_elems) == (3, 128)
    bad = WeightStore(write_model(tmp_path / "bad", {"s.safetensors": {"layer.weight": w, "layer.scales": s3,
                                                                       "layer.biases": s2}}))
    with pytest.raises(QmError, match="INVALID_TENSOR"):
        bad.upload_q4(rt, "layer.weight")
