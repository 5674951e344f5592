"""GPU parity of the MLX affine-Q4 projections against the CPU oracle.

Ports metal_runtime.rs tests q4_affine_matvec_matches_cpu_reference (:9365),
mapped_q4_batch_reuses_one_input_without_changing_results (:9685),
mapped_q4_matmul_batch_matches_each_prompt_row (:9766),
batch_simd_q4_matmul_short_batch_matches_cpu_reference (:9812) and
fused_q4_mlp_batch_matches_cpu_reference (:10726), plus seeded
BASELINE-shape cases.  Tolerance: bf16 outputs within 1e-4 of max |ref|
beyond the bf16 output rounding (fp64-accumulated oracle).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from gpu_util import assert_bf16_close, bf16_dev_to_f32, empty_bf16, to_dev, tuned
from qm38 import QmError, synth

pytestmark = pytest.mark.gpu


def _upload(dev, packed, s, b):
    return to_dev(packed, dev), to_dev(s, dev), to_dev(b, dev)


def _project(rt, dev, mats, x_bits, M):
    import qm38
    K = x_bits.shape[-1]
    xd = to_dev(x_bits, dev)
    devm = [_upload(dev, *m) for m in mats]
    jobs = [qm38.Runtime.job(w, s, b, m[0].shape[0]) for (w, s, b), m in zip(devm, mats)]
    outs = [empty_bf16((M, m[0].shape[0]), dev) for m in mats]
    rt.q4_project(jobs, xd, K, M, outs)
    return [bf16_dev_to_f32(o) for o in outs]


def test_reference_vectors_k128_n5(rt, torch_dev):
    # metal_runtime.rs:9332-9362: ramp input, nibbles (i*7+3)%16, scale/bias tables.
    K, N = 128, 5
    x = ((np.arange(K) % 17) - 8.0) * 0.125
    q = ((np.arange(N * K) * 7 + 3) % 16).astype(np.uint8).reshape(N, K)
    sv = [0.125, -0.0625, 0.25, 0.03125, -0.125, 0.0625]
    bv = [0.03125, -0.015625, 0.0625, 0.125, -0.03125, 0.0]
    s = synth.f32_to_bf16(np.array([sv[i % 6] for i in range(N * 2)], np.float32)).reshape(N, 2)
    b = synth.f32_to_bf16(np.array([bv[i % 6] for i in range(N * 2)], np.float32)).reshape(N, 2)
    xb = synth.f32_to_bf16(x.astype(np.float32))[None]
    mat = (synth.pack_q4(q), s, b)
    (got,) = _project(rt, torch_dev, [mat], xb, 1)
    ref = oracle.q4_project(xb, *mat)
    assert_bf16_close(got, ref, what="k128n5")
    # reference tolerance: abs < 1e-3 against fp32 outputs (bf16 here: 1 ulp slack)
    assert np.max(np.abs(got - ref)) < 1e-3 + np.max(np.abs(ref)) * 2 ** -8


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 13, 16])
@pytest.mark.parametrize("N,K", [(40, 256), (257, 512), (96, 192), (1024, 1024)])
def test_short_batch_matches_oracle(rt, torch_dev, M, N, K):
    rng = np.random.default_rng(1000 + M * 31 + N + K)
    mat = synth.q4_matrix(rng, N, K)
    xb = synth.bf16_normal(rng, (M, K))
    (got,) = _project(rt, torch_dev, [mat], xb, M)
    ref = oracle.q4_project(xb, *mat)
    assert_bf16_close(got, ref, what=f"M{M} N{N} K{K}")


def test_batch_of_jobs_reuses_one_input(rt, torch_dev):
    # One activation, several projections of different heights in one launch
    # must equal each projection run alone (metal_runtime.rs:9685).
    rng = np.random.default_rng(7)
    K = 512
    mats = [synth.q4_matrix(rng, n, K) for n in (64, 200, 33, 512)]
    for M in (1, 4, 8):
        xb = synth.bf16_normal(rng, (M, K))
        together = _project(rt, torch_dev, mats, xb, M)
        for mat, got in zip(mats, together):
            (alone,) = _project(rt, torch_dev, [mat], xb, M)
            np.testing.assert_array_equal(got, alone)
            assert_bf16_close(got, oracle.q4_project(xb, *mat))


def test_matmul_rows_equal_per_row_matvec(rt, torch_dev):
    # metal_runtime.rs:9766: a multi-row call equals one call per row.
    rng = np.random.default_rng(11)
    K, N, M = 384, 130, 6
    mat = synth.q4_matrix(rng, N, K)
    xb = synth.bf16_normal(rng, (M, K))
    (batch,) = _project(rt, torch_dev, [mat], xb, M)
    for m in range(M):
        (row,) = _project(rt, torch_dev, [mat], xb[m:m + 1], 1)
        assert_bf16_close(batch[m:m + 1], row.astype(np.float64))


def test_identity_bias_cancels(rt, torch_dev):
    # q = 8 everywhere and b = -8 s: every weight is exactly 0, so y is 0 up to
    # the fp32 rounding of the kernel's s*sum((128+q)x) + (b-128s)*sum(x) form.
    rng = np.random.default_rng(3)
    N, K = 64, 256
    packed = np.full((N, K // 8), 0x88888888, np.uint32)
    s = synth.f32_to_bf16(rng.uniform(0.005, 0.02, (N, K // 64)).astype(np.float32))
    b = synth.f32_to_bf16(-8 * synth.bf16_to_f32(s))
    xb = synth.bf16_normal(rng, (4, K))
    (got,) = _project(rt, torch_dev, [(packed, s, b)], xb, 4)
    bound = 1e-5 * np.max(synth.bf16_to_f32(s)) * np.sum(np.abs(synth.bf16_to_f32(xb)), axis=1).max() * 136
    assert np.max(np.abs(got)) <= bound


@pytest.mark.parametrize("M", [1, 4, 8])
def test_swiglu_pair_and_mlp(rt, torch_dev, M):
    import qm38
    rng = np.random.default_rng(50 + M)
    K, I = 512, 768
    gate = synth.q4_matrix(rng, I, K)
    up = synth.q4_matrix(rng, I, K)
    down = synth.q4_matrix(rng, K, I)
    xb = synth.bf16_normal(rng, (M, K))
    g_ref = oracle.q4_project(xb, *gate)
    u_ref = oracle.q4_project(xb, *up)
    h_ref = oracle.swiglu(g_ref, u_ref)
    dg, du, dd = (_upload(torch_dev, *m) for m in (gate, up, down))
    jg = qm38.Runtime.job(*dg, I)
    ju = qm38.Runtime.job(*du, I)
    jd = qm38.Runtime.job(*dd, K)
    xd = to_dev(xb, torch_dev)
    h = empty_bf16((M, I), torch_dev)
    rt.q4_swiglu(jg, ju, xd, K, M, h)
    h_got = bf16_dev_to_f32(h)
    assert_bf16_close(h_got, h_ref, what="swiglu h")
    y = empty_bf16((M, K), torch_dev)
    rt.q4_mlp(jg, ju, jd, xd, K, M, y)
    # down consumes the bf16 h the kernel wrote
    y_ref = oracle.q4_project(synth.f32_to_bf16(h_got), *down)
    assert_bf16_close(bf16_dev_to_f32(y), y_ref, what="mlp y")
    # and against the all-fp32 chain (h not rounded): rounding h to bf16 is
    # the only extra error
    y_ref32 = oracle.q4_project(synth.f32_to_bf16(h_ref), *down)
    assert_bf16_close(bf16_dev_to_f32(y), y_ref32, rel=1e-3, what="mlp y vs unrounded-h chain")


@pytest.mark.parametrize("M", [1, 4, 8])
def test_decode_set_27b_shapes(rt, torch_dev, M):
    # QKV 5120->10240, gate/up 5120->2x17408, down 17408->5120.
    import qm38
    rng = np.random.default_rng(2024 + M)
    H, I, QKV = 5120, 17408, 10240
    qkv = synth.q4_matrix(rng, QKV, H)
    xb = synth.bf16_normal(rng, (M, H))
    (got,) = _project(rt, torch_dev, [qkv], xb, M)
    assert_bf16_close(got, oracle.q4_project(xb, *qkv), what="qkv")
    gate = synth.q4_matrix(rng, I, H)
    up = synth.q4_matrix(rng, I, H)
    dg, du = _upload(torch_dev, *gate), _upload(torch_dev, *up)
    h = empty_bf16((M, I), torch_dev)
    rt.q4_swiglu(qm38.Runtime.job(*dg, I), qm38.Runtime.job(*du, I), to_dev(xb, torch_dev), H, M, h)
    h_got = bf16_dev_to_f32(h)
    h_ref = oracle.swiglu(oracle.q4_project(xb, *gate), oracle.q4_project(xb, *up))
    assert_bf16_close(h_got, h_ref, what="gate/up")
    down = synth.q4_matrix(rng, H, I)
    hb = synth.f32_to_bf16(h_got)
    (y,) = _project(rt, torch_dev, [down], hb, M)
    assert_bf16_close(y, oracle.q4_project(hb, *down), what="down")


@pytest.mark.parametrize("nt,rpw", [(1, 16), (1, 13), (1, 10), (1, 8), (2, 32), (2, 20), (2, 17)])
@pytest.mark.parametrize("M", [1, 3, 8])
def test_rows_per_workgroup(torch_dev, nt, rpw, M):
    """Workgroups owning fewer rows than their 16-row tiles (the planner's
    balancing choice) mask the rest; forced here for several row counts that
    do not divide the projection heights, with several jobs in one launch and
    a SwiGLU pair.  (The MFMA decode kernel: the streaming kernels, which
    take up to eight rows by default, are switched off.)"""
    import qm38
    with tuned(QM38_Q4_NT=nt, QM38_Q4_RPW=rpw, QM38_Q4_STREAM=0, QM38_Q4_MMA_LO=0, QM38_Q4_MMA_K=0) as rt:
        rng = np.random.default_rng(300 + nt * 50 + rpw + M)
        K = 1024
        mats = [synth.q4_matrix(rng, n, K) for n in (200, 37, 512)]
        xb = synth.bf16_normal(rng, (M, K))
        for mat, got in zip(mats, _project(rt, torch_dev, mats, xb, M)):
            assert_bf16_close(got, oracle.q4_project(xb, *mat), what=f"rows {mat[0].shape[0]}")
        I = 333
        gate, up = synth.q4_matrix(rng, I, K), synth.q4_matrix(rng, I, K)
        dg, du = _upload(torch_dev, *gate), _upload(torch_dev, *up)
        h = empty_bf16((M, I), torch_dev)
        rt.q4_swiglu(qm38.Runtime.job(*dg, I), qm38.Runtime.job(*du, I), to_dev(xb, torch_dev), K, M, h)
        h_ref = oracle.swiglu(oracle.q4_project(xb, *gate), oracle.q4_project(xb, *up))
        assert_bf16_close(bf16_dev_to_f32(h), h_ref, what="swiglu")


def test_config1_4096(rt, torch_dev):
    rng = np.random.default_rng(1)
    mat = synth.q4_matrix(rng, 4096, 4096)
    xb = synth.bf16_normal(rng, (1, 4096))
    (got,) = _project(rt, torch_dev, [mat], xb, 1)
    assert_bf16_close(got, oracle.q4_project(xb, *mat), what="cfg1")


def test_rejects_incomplete_group(rt, torch_dev):
    # metal_runtime.rs:11806 q4_affine_matvec_rejects_incomplete_group
    import qm38
    rng = np.random.default_rng(0)
    mat = synth.q4_matrix(rng, 8, 64)
    w, s, b = _upload(torch_dev, *mat)
    x = to_dev(synth.bf16_normal(rng, (1, 64)), torch_dev)
    out = empty_bf16((1, 8), torch_dev)
    with pytest.raises(QmError) as e:
        rt.q4_project([qm38.Runtime.job(w, s, b, 8)], x, 63, 1, [out])
    assert e.value.status == "QM_ERR_INPUT_NOT_GROUPED"
    with pytest.raises(QmError) as e:
        rt.q4_project([qm38.Runtime.job(w, s, b, 0)], x, 64, 1, [out])
    assert e.value.status == "QM_ERR_EMPTY_DIMENSION"


def _argmax_ref(y: np.ndarray) -> np.ndarray:
    """qwen38_argmax_rows (qwen38.metal:4202-4244): largest value, lowest index
    on ties, NaN never winning (an all-NaN row gives 0)."""
    out = np.zeros(y.shape[0], np.uint32)
    for m in range(y.shape[0]):
        row = np.where(np.isnan(y[m]), -np.inf, y[m])
        if np.all(np.isnan(y[m])):
            continue
        out[m] = int(np.flatnonzero(row == row.max())[0])
    return out


def _argmax(rt, dev, mat, xb):
    import torch
    import qm38
    w, s, b = _upload(dev, *mat)
    M = xb.shape[0]
    ids = torch.full((M,), -1, dtype=torch.int32, device=dev)
    rt.q4_affine_argmax(qm38.Runtime.job(w, s, b, mat[0].shape[0]), to_dev(xb, dev), xb.shape[1], M, ids)
    return from_dev_u32(ids)


def from_dev_u32(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("M", [1, 3, 16, 37])
def test_argmax_matches_oracle(rt, torch_dev, M):
    # q4_affine_argmax_mapped_batch (metal_runtime.rs:3797): the greedy token
    # of every row.  The kernel's fp32 sums and the fp64 oracle may order a
    # near-tie differently, so a row must pick the oracle's winner unless the
    # runner-up lies within the fp32 error bound; then its pick must be one of
    # those near-maximal rows.  M = 37 runs in chunks of 16 rows.
    rng = np.random.default_rng(4100 + M)
    N, K = 1000, 512
    mat = synth.q4_matrix(rng, N, K)
    xb = synth.bf16_normal(rng, (M, K))
    got = _argmax(rt, torch_dev, mat, xb)
    ref = oracle.q4_project(xb, *mat)
    tol = 1e-5 * np.max(np.abs(ref), axis=1)
    for m in range(M):
        near = np.flatnonzero(ref[m] >= ref[m].max() - tol[m])
        assert got[m] in near, f"row {m}: picked {got[m]}, oracle winners {near}"
        if len(near) == 1:
            assert got[m] == near[0]


def test_argmax_ties_nan_and_empty_rows(rt, torch_dev):
    # Identical rows give bit-identical logits: the lowest index wins
    # (qwen38.metal:4218-4221).  A NaN scale makes its row NaN, which never
    # wins; an all-NaN activation row makes every logit NaN and gives 0.
    rng = np.random.default_rng(77)
    N, K = 517, 256
    w, s, b = synth.q4_matrix(rng, N, K)
    xb = synth.bf16_normal(rng, (3, K))
    xb[1] = 0x7FC0  # bf16 NaN
    r = int(np.argmax(oracle.q4_project(xb[:1], w, s, b)[0]))
    for j in (3, N - 1, (r + 200) % N):
        w[j], s[j], b[j] = w[r], s[r], b[r]
    s[0] = 0x7FC0
    got = _argmax(rt, torch_dev, (w, s, b), xb)
    y = oracle.q4_project(xb, w, s, b)
    assert np.isnan(y[0, 0]) and np.all(np.isnan(y[1]))
    want = _argmax_ref(y)
    assert want[0] == 3 and want[1] == 0
    assert got[0] == 3 and got[1] == 0
    assert got[2] == want[2] or y[2, got[2]] >= y[2].max() - 1e-5 * np.max(np.abs(y[2]))
    # the same rows through the plain projection: the tie is exact in the kernel too
    (proj,) = _project(rt, torch_dev, [(w, s, b)], xb[:1], 1)
    assert proj[0, 3] == proj[0, r] == proj[0, N - 1]


def test_projection_ranges_are_checked(rt, torch_dev):
    # validate_mapped_q4_affine_shape (metal_runtime.rs:8854-8898): a tensor
    # running past its allocation is refused before anything is launched, and
    # a pointer inside no allocation is an invalid offset.  Sizes are whole
    # 4 KiB pages so the allocation's length is exactly what was asked for.
    import qm38
    rng = np.random.default_rng(8)
    N, K = 64, 1024
    w, s, b = synth.q4_matrix(rng, N, K)
    dw, ds, db = rt.device_buffer(w), rt.device_buffer(s), rt.device_buffer(b)
    short_w = rt.device_buffer(w[:56])  # 28672 B of the 32768 needed
    x = to_dev(synth.bf16_normal(rng, (1, K)), torch_dev)
    out = empty_bf16((1, N), torch_dev)
    rt.q4_project([qm38.Runtime.job(dw, ds, db, N)], x, K, 1, [out])  # in range
    with pytest.raises(QmError) as e:
        rt.q4_project([qm38.Runtime.job(short_w, ds, db, N)], x, K, 1, [out])
    assert e.value.status == "QM_ERR_MAPPED_TENSOR_OUT_OF_RANGE"
    with pytest.raises(QmError) as e:  # one row too many for every tensor
        rt.q4_project([qm38.Runtime.job(dw, ds, db, N + 1)], x, K, 1, [empty_bf16((1, N + 1), torch_dev)])
    assert e.value.status == "QM_ERR_MAPPED_TENSOR_OUT_OF_RANGE"
    host = np.zeros(1 << 16, np.uint8)  # ordinary host memory: no device allocation
    with pytest.raises(QmError) as e:
        rt.q4_project([qm38.Runtime.job(host.ctypes.data, ds, db, N)], x, K, 1, [out])
    assert e.value.status == "QM_ERR_INVALID_BUFFER_OFFSET"
    small_out = rt.device_buffer(nbytes=64)
    with pytest.raises(QmError) as e:  # the output needs 128 B
        rt.q4_project([qm38.Runtime.job(dw, ds, db, N)], x, K, 1, [small_out])
    assert e.value.status == "QM_ERR_MAPPED_TENSOR_OUT_OF_RANGE"
    with pytest.raises(QmError) as e:
        rt.q4_affine_argmax(qm38.Runtime.job(short_w, ds, db, N), x, K, 1, out)
    assert e.value.status == "QM_ERR_MAPPED_TENSOR_OUT_OF_RANGE"


def test_mapped_job_from_one_buffer(rt, torch_dev):
    # MappedQ4AffineJob: weights, scales and biases at byte offsets of one
    # checkpoint-like allocation give the same projection as separate tensors.
    import qm38
    rng = np.random.default_rng(9)
    N, K = 96, 512
    w, s, b = synth.q4_matrix(rng, N, K)
    blob = np.concatenate([np.zeros(256, np.uint8), w.view(np.uint8).ravel(), s.view(np.uint8).ravel(),
                           np.zeros(8, np.uint8), b.view(np.uint8).ravel()])
    buf = rt.device_buffer(blob)
    whole = (buf.ptr, blob.nbytes)
    off_w, off_s = 256, 256 + w.nbytes
    off_b = off_s + s.nbytes + 8
    job = qm38.Runtime.mapped_job(whole, off_w, whole, off_s, whole, off_b, N, K)
    xb = synth.bf16_normal(rng, (2, K))
    out = empty_bf16((2, N), torch_dev)
    rt.q4_project([job], to_dev(xb, torch_dev), K, 2, [out])
    assert_bf16_close(bf16_dev_to_f32(out), oracle.q4_project(xb, w, s, b), what="mapped")
    with pytest.raises(QmError) as e:
        qm38.Runtime.mapped_job(whole, off_w, whole, off_s, whole, off_b + 8, N, K)
    assert e.value.status == "QM_ERR_MAPPED_TENSOR_OUT_OF_RANGE"
    with pytest.raises(QmError) as e:
        qm38.Runtime.mapped_job(whole, blob.nbytes + 1, whole, off_s, whole, off_b, N, K)
    assert e.value.status == "QM_ERR_INVALID_BUFFER_OFFSET"


@pytest.mark.parametrize("M", [2])
@pytest.mark.parametrize("K", [192, 1024, 5120, 8256, 17408, 20544])
def test_few_rows_streaming(torch_dev, M, K):
    """Two activation rows on the streaming kernel (one chunk per wave, K in
    balanced parts of at most 8 waves whose fp32 sums the last part adds;
    K = 192 and 8256 end inside a chunk; long K kept off the MFMA streaming
    kernel with QM38_Q4_MMA_K=0): plain jobs of several heights and a SwiGLU
    pair in one launch each match the oracle row by row, repeated calls are
    bit-identical, and the result equals the MFMA decode kernel's within the
    same bar."""
    with tuned(QM38_Q4_MMA_K=0) as rt:
        _few_rows_streaming(rt, torch_dev, M, K)


def _few_rows_streaming(rt, torch_dev, M, K):
    import qm38
    rng = np.random.default_rng(K * 10 + M)
    mats = [synth.q4_matrix(rng, n, K) for n in (300, 37)]
    xb = synth.bf16_normal(rng, (M, K))
    got1 = _project(rt, torch_dev, mats, xb, M)
    got2 = _project(rt, torch_dev, mats, xb, M)
    for mat, g1, g2 in zip(mats, got1, got2):
        assert_bf16_close(g1, oracle.q4_project(xb, *mat), what=f"M={M} K={K} rows {mat[0].shape[0]}")
        assert np.array_equal(g1, g2)
    gate, up = synth.q4_matrix(rng, 90, K), synth.q4_matrix(rng, 90, K)
    dg, du = _upload(torch_dev, *gate), _upload(torch_dev, *up)
    jg, ju = qm38.Runtime.job(*dg, 90), qm38.Runtime.job(*du, 90)
    h = empty_bf16((M, 90), torch_dev)
    rt.q4_swiglu(jg, ju, to_dev(xb, torch_dev), K, M, h)
    h_ref = oracle.swiglu(oracle.q4_project(xb, *gate), oracle.q4_project(xb, *up))
    assert_bf16_close(bf16_dev_to_f32(h), h_ref, what=f"M={M} K={K} swiglu")
    with tuned(QM38_Q4_STREAM=0, QM38_Q4_MMA_LO=0, QM38_Q4_MMA_K=0) as mrt:
        for mat, g1 in zip(mats, _project(mrt, torch_dev, mats, xb, M)):
            assert_bf16_close(g1, oracle.q4_project(xb, *mat), what=f"decode kernel M={M} K={K}")


@pytest.mark.parametrize("K", [16448, 17408, 20544])
def test_single_row_k_parts(rt, torch_dev, K):
    """One activation row with K beyond 16384: the streaming kernel splits K
    over several workgroups (parts of 5120 elements, the last one shorter,
    here also ending inside a 512-element chunk for K = 16448 and 20544) and
    the last part to finish adds the fp32 partial rows in part order.  Plain
    jobs of several heights, a SwiGLU pair and the argmax all match the
    oracle, and repeated calls are bit-identical."""
    import torch
    import qm38
    rng = np.random.default_rng(K)
    mats = [synth.q4_matrix(rng, n, K) for n in (300, 37)]
    xb = synth.bf16_normal(rng, (1, K))
    got1 = _project(rt, torch_dev, mats, xb, 1)
    got2 = _project(rt, torch_dev, mats, xb, 1)
    for mat, g1, g2 in zip(mats, got1, got2):
        assert_bf16_close(g1, oracle.q4_project(xb, *mat), what=f"K={K} rows {mat[0].shape[0]}")
        assert np.array_equal(g1, g2)
    gate, up = synth.q4_matrix(rng, 90, K), synth.q4_matrix(rng, 90, K)
    dg, du = _upload(torch_dev, *gate), _upload(torch_dev, *up)
    h = empty_bf16((1, 90), torch_dev)
    rt.q4_swiglu(qm38.Runtime.job(*dg, 90), qm38.Runtime.job(*du, 90), to_dev(xb, torch_dev), K, 1, h)
    h_ref = oracle.swiglu(oracle.q4_project(xb, *gate), oracle.q4_project(xb, *up))
    assert_bf16_close(bf16_dev_to_f32(h), h_ref, what=f"K={K} swiglu")
    ids = _argmax(rt, torch_dev, mats[0], xb)
    ref = oracle.q4_project(xb, *mats[0])[0]
    assert ref[ids[0]] >= ref.max() - 1e-5 * np.max(np.abs(ref))


def test_project_set_mixes_plain_and_pairs(rt, torch_dev):
    """qm_q4_project_set: plain projections and SwiGLU pairs from one
    activation, in one launch for one or two rows and prefill rows (the GEMM
    takes both tile kinds), one launch for 1..8 rows (the streaming kernels), as separate launches for 9..16 rows; each output
    matches the oracle, and a pair's equals its own call's where both run the
    same kernel plan."""
    import qm38
    rng = np.random.default_rng(31)
    K = 1024
    for M in (1, 2, 3, 40):
        a, g, u, b = (synth.q4_matrix(rng, n, K) for n in (200, 96, 96, 40))
        da, dg, du, db = (_upload(torch_dev, *m) for m in (a, g, u, b))
        ja, jg, ju, jb = (qm38.Runtime.job(*d, m[0].shape[0]) for d, m in zip((da, dg, du, db), (a, g, u, b)))
        xb = synth.bf16_normal(rng, (M, K))
        xd = to_dev(xb, torch_dev)
        outs = [empty_bf16((M, 200), torch_dev), empty_bf16((M, 96), torch_dev), empty_bf16((M, 40), torch_dev)]
        rt.q4_project_set([ja, jg, jb], [None, ju, None], xd, K, M, outs)
        assert_bf16_close(bf16_dev_to_f32(outs[0]), oracle.q4_project(xb, *a), what=f"set plain M={M}")
        h_ref = oracle.swiglu(oracle.q4_project(xb, *g), oracle.q4_project(xb, *u))
        assert_bf16_close(bf16_dev_to_f32(outs[1]), h_ref, what=f"set pair M={M}")
        assert_bf16_close(bf16_dev_to_f32(outs[2]), oracle.q4_project(xb, *b), what=f"set plain 2 M={M}")
        if M > 16:
            continue  # the GEMM's plan (and so its sum order) follows the launch's tile count
        h = empty_bf16((M, 96), torch_dev)
        rt.q4_swiglu(jg, ju, xd, K, M, h)
        assert np.array_equal(bf16_dev_to_f32(h), bf16_dev_to_f32(outs[1]))


@pytest.mark.parametrize("C", [4, 8])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("K", [192, 1024, 5120, 6208, 17408])
def test_mma_streaming_rows(torch_dev, M, K, C):
    """The MFMA streaming kernel (q4_mma.hip) forced for 1..8 activation rows
    (QM38_Q4_MMA_LO=1, QM38_Q4_MMA_HI=8, the single-row kernel off):
    128-element spans in pairs, A rows (span, group, activation row), two A
    halves beyond four rows; K = 192 and 6208 end inside a span, 17408 runs in
    K parts whose fp32 sums the last part adds.
    Plain jobs of several heights (not multiples of 16), a SwiGLU pair and a
    mixed set (one launch, 32-row blocks) match the oracle row by row, and
    repeated calls are bit-identical."""
    import qm38
    rng = np.random.default_rng(K * 100 + M)
    mats = [synth.q4_matrix(rng, n, K) for n in (300, 37)]
    xb = synth.bf16_normal(rng, (M, K))
    gate, up = synth.q4_matrix(rng, 90, K), synth.q4_matrix(rng, 90, K)
    h_ref = oracle.swiglu(oracle.q4_project(xb, *gate), oracle.q4_project(xb, *up))
    with tuned(QM38_Q4_MMA_LO=1, QM38_Q4_MMA_HI=8, QM38_Q4_STREAM=0, QM38_Q4_MMA_C=C) as mrt:
        got1 = _project(mrt, torch_dev, mats, xb, M)
        got2 = _project(mrt, torch_dev, mats, xb, M)
        for mat, g1, g2 in zip(mats, got1, got2):
            assert_bf16_close(g1, oracle.q4_project(xb, *mat), what=f"M={M} K={K} rows {mat[0].shape[0]}")
            assert np.array_equal(g1, g2)
        dg, du = _upload(torch_dev, *gate), _upload(torch_dev, *up)
        jg, ju = qm38.Runtime.job(*dg, 90), qm38.Runtime.job(*du, 90)
        xd = to_dev(xb, torch_dev)
        h = empty_bf16((M, 90), torch_dev)
        mrt.q4_swiglu(jg, ju, xd, K, M, h)
        assert_bf16_close(bf16_dev_to_f32(h), h_ref, what=f"M={M} K={K} swiglu")
        dm = _upload(torch_dev, *mats[0])
        jm = qm38.Runtime.job(*dm, 300)
        outs = [empty_bf16((M, 300), torch_dev), empty_bf16((M, 90), torch_dev)]
        mrt.q4_project_set([jm, jg], [None, ju], xd, K, M, outs)
        assert np.array_equal(bf16_dev_to_f32(outs[0]), got1[0])
        assert np.array_equal(bf16_dev_to_f32(outs[1]), bf16_dev_to_f32(h))
