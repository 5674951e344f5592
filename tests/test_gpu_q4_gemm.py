"""GPU parity of the Q4 prefill GEMM (M > 16) against the CPU oracle.

Ports mapped_q4_matmul_batch_matches_each_prompt_row (metal_runtime.rs:9766),
simdgroup_q4_matmul_batch_matches_cpu_reference (:10560),
wide_simdgroup_q4_matmul_batch_matches_cpu_reference (:10620) and
fused_q4_mlp_batch_matches_cpu_reference at M = 256 (:10726), plus the
BASELINE prefill shapes.  The kernel computes like the reference's prefill
path: fp16(q*s + b) weights, fp16 activations, fp32 accumulation; the
oracle is exact (fp64).  Bar: bf16 outputs within 1e-4 of max|ref| beyond
the bf16 output rounding (tests/gpu_util.py).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from gpu_util import assert_bf16_close, bf16_dev_to_f32, empty_bf16, to_dev, tuned
from qm38 import synth

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


@pytest.mark.parametrize("M", [17, 64, 255, 256, 300, 512])
@pytest.mark.parametrize("N,K", [(40, 256), (257, 512), (1024, 1024), (640, 192)])
def test_gemm_matches_oracle(rt, torch_dev, M, N, K):
    rng = np.random.default_rng(7000 + M * 13 + N + K)
    mat = synth.q4_matrix(rng, N, K)
    xb = synth.bf16_normal(rng, (M, K))
    (got,) = _project(rt, torch_dev, [mat], xb, M)
    assert_bf16_close(got, oracle.q4_project(xb, *mat), what=f"M{M} N{N} K{K}")


def test_jobs_in_one_launch_equal_jobs_alone(rt, torch_dev):
    rng = np.random.default_rng(8)
    K, M = 512, 300
    mats = [synth.q4_matrix(rng, n, K) for n in (64, 200, 33, 512)]
    xb = synth.bf16_normal(rng, (M, K))
    together = _project(rt, torch_dev, mats, xb, M)
    for mat, got in zip(mats, together):
        (alone,) = _project(rt, torch_dev, [mat], xb, M)
        np.testing.assert_array_equal(got, alone)
        assert_bf16_close(got, oracle.q4_project(xb, *mat))


def test_rows_do_not_interact(rt, torch_dev):
    # metal_runtime.rs:9766: each prompt row equals its own projection; here a
    # row of a 300-row GEMM equals the same row inside a different batch.
    rng = np.random.default_rng(12)
    K, N = 1024, 384
    mat = synth.q4_matrix(rng, N, K)
    xb = synth.bf16_normal(rng, (300, K))
    (full,) = _project(rt, torch_dev, [mat], xb, 300)
    perm = rng.permutation(300)[:40]
    (sub,) = _project(rt, torch_dev, [mat], xb[perm], 40)
    np.testing.assert_array_equal(full[perm], sub)


def test_identity_weights_are_exactly_zero(rt, torch_dev):
    # q = 8, b = -8 s: fp16(8 s - 8 s) = 0 for every weight, so Y = 0 exactly.
    rng = np.random.default_rng(3)
    N, K, M = 300, 512, 77
    packed = np.full((N, K // 8), 0x88888888, np.uint32)
    s = synth.f32_to_bf16(rng.uniform(0.005, 0.02, (N, K // 64)).astype(np.float32))
    b = synth.f32_to_bf16(-8 * synth.bf16_to_f32(s))
    xb = synth.bf16_normal(rng, (M, K))
    (got,) = _project(rt, torch_dev, [(packed, s, b)], xb, M)
    assert np.all(got == 0.0)


def test_constant_nibble_closed_form(rt, torch_dev):
    # q = c everywhere: y[m][n] = sum_g (s_g c + b_g) * sum_{i in g} x[m][i].
    rng = np.random.default_rng(4)
    N, K, M, c = 96, 640, 40, 11
    packed = np.full((N, K // 8), int("0x" + f"{c:x}" * 8, 16), np.uint32)
    s = synth.f32_to_bf16(rng.uniform(0.005, 0.02, (N, K // 64)).astype(np.float32))
    b = synth.f32_to_bf16(rng.normal(0, 0.05, (N, K // 64)).astype(np.float32))
    xb = synth.bf16_normal(rng, (M, K))
    (got,) = _project(rt, torch_dev, [(packed, s, b)], xb, M)
    xs = synth.bf16_to_f32(xb).astype(np.float64).reshape(M, K // 64, 64).sum(-1)
    wg = synth.bf16_to_f32(s).astype(np.float64) * c + synth.bf16_to_f32(b).astype(np.float64)
    # The kernel's weights are fp16(q s + b) (the reference's prefill
    # numerics); the closed form uses the exact s c + b: about 2e-4 apart.
    assert_bf16_close(got, xs @ wg.T, rel=1e-3, what="constant nibble")


def test_activation_beyond_fp16_range_saturates(rt, torch_dev):
    # The GEMM stages activations in fp16; a bf16 value beyond +-65504 is
    # clamped to +-65504 instead of becoming an infinity, so the result equals
    # the exact projection of the clamped input and every output stays finite.
    rng = np.random.default_rng(21)
    N, K, M = 192, 512, 40
    mat = synth.q4_matrix(rng, N, K)
    xf = synth.bf16_to_f32(synth.bf16_normal(rng, (M, K)))
    xf[3, 17] = 1.0e5
    xf[9, 300] = -3.0e6
    xf[20, :8] = 7.0e4
    xb = synth.f32_to_bf16(xf)
    (got,) = _project(rt, torch_dev, [mat], xb, M)
    assert np.all(np.isfinite(got))
    # 65504 is not a bf16 value; by linearity P(clamp(x)) = P(x') - P(d), where
    # x' holds +-65536 at the clamped places and d holds +-32 there (both exact
    # in bf16).
    xv = synth.bf16_to_f32(xb)
    big = np.abs(xv) > 65504.0
    xp = np.where(big, np.sign(xv) * 65536.0, xv).astype(np.float32)
    d = np.where(big, np.sign(xv) * 32.0, 0.0).astype(np.float32)
    want = (oracle.q4_project(synth.f32_to_bf16(xp), *mat).astype(np.float64)
            - oracle.q4_project(synth.f32_to_bf16(d), *mat))
    for m in range(M):  # row by row: the saturated rows' scale would hide the rest
        assert_bf16_close(got[m], want[m], what=f"saturated activations, row {m}")


@pytest.mark.parametrize("M", [64, 256, 300])
def test_swiglu_and_mlp(rt, torch_dev, M):
    # fused_q4_mlp_batch_matches_cpu_reference (metal_runtime.rs:10726) at M = 256.
    import qm38
    rng = np.random.default_rng(60 + M)
    K, I = 512, 768
    gate = synth.q4_matrix(rng, I, K)
    up = synth.q4_matrix(rng, I, K)
    down = synth.q4_matrix(rng, K, I)
    xb = synth.bf16_normal(rng, (M, K))
    h_ref = oracle.swiglu(oracle.q4_project(xb, *gate), oracle.q4_project(xb, *up))
    dg, du, dd = (_upload(torch_dev, *m) for m in (gate, up, down))
    jg, ju, jd = qm38.Runtime.job(*dg, I), qm38.Runtime.job(*du, I), qm38.Runtime.job(*dd, K)
    xd = to_dev(xb, torch_dev)
    h = empty_bf16((M, I), torch_dev)
    rt.q4_swiglu(jg, ju, xd, K, M, h)
    h_got = bf16_dev_to_f32(h)
    assert_bf16_close(h_got, h_ref, what="swiglu h")
    y = empty_bf16((M, K), torch_dev)
    rt.q4_mlp(jg, ju, jd, xd, K, M, y)
    y_ref = oracle.q4_project(synth.f32_to_bf16(h_got), *down)
    assert_bf16_close(bf16_dev_to_f32(y), y_ref, what="mlp y")


@pytest.mark.parametrize("M", [512, 2048])
def test_prefill_27b_shapes(rt, torch_dev, M):
    # QKV 5120->10240, gate/up 5120->2x17408, down 17408->5120.
    # Rows are independent, so the oracle checks a seeded sample of 24 rows.
    import qm38
    rng = np.random.default_rng(3000 + M)
    H, I, QKV = 5120, 17408, 10240
    xb = synth.bf16_normal(rng, (M, H))
    rows = np.sort(np.concatenate([[0, M - 1], rng.choice(np.arange(1, M - 1), 22, replace=False)]))
    qkv = synth.q4_matrix(rng, QKV, H)
    (got,) = _project(rt, torch_dev, [qkv], xb, M)
    assert_bf16_close(got[rows], oracle.q4_project(xb[rows], *qkv), what="qkv")
    del qkv
    gate, up = synth.q4_matrix(rng, I, H), synth.q4_matrix(rng, I, H)
    dg, du = _upload(torch_dev, *gate), _upload(torch_dev, *up)
    h = empty_bf16((M, I), torch_dev)
    rt.q4_swiglu(qm38.Runtime.job(*dg, I), qm38.Runtime.job(*du, I), to_dev(xb, torch_dev), H, M, h)
    h_got = bf16_dev_to_f32(h)
    h_ref = oracle.swiglu(oracle.q4_project(xb[rows], *gate), oracle.q4_project(xb[rows], *up))
    assert_bf16_close(h_got[rows], h_ref, what="gate/up")
    del gate, up, dg, du
    down = synth.q4_matrix(rng, H, I)
    hb = synth.f32_to_bf16(h_got)
    (y,) = _project(rt, torch_dev, [down], hb, M)
    assert_bf16_close(y[rows], oracle.q4_project(hb[rows], *down), what="down")


@pytest.mark.parametrize("M", [33, 300])
def test_split_k_swiglu_and_determinism(rt, torch_dev, M):
    # K = 2048 (32 groups) with few output tiles: the launch splits K across
    # workgroups, and the last slice of each tile adds the slices in a fixed
    # order, so two calls agree bit for bit.
    import qm38
    rng = np.random.default_rng(90 + M)
    K, I = 2048, 384
    gate = synth.q4_matrix(rng, I, K)
    up = synth.q4_matrix(rng, I, K)
    xb = synth.bf16_normal(rng, (M, K))
    h_ref = oracle.swiglu(oracle.q4_project(xb, *gate), oracle.q4_project(xb, *up))
    dg, du = _upload(torch_dev, *gate), _upload(torch_dev, *up)
    jg, ju = qm38.Runtime.job(*dg, I), qm38.Runtime.job(*du, I)
    xd = to_dev(xb, torch_dev)
    h1, h2 = empty_bf16((M, I), torch_dev), empty_bf16((M, I), torch_dev)
    rt.q4_swiglu(jg, ju, xd, K, M, h1)
    rt.q4_swiglu(jg, ju, xd, K, M, h2)
    got = bf16_dev_to_f32(h1)
    assert_bf16_close(got, h_ref, what="split-K swiglu")
    assert np.array_equal(got, bf16_dev_to_f32(h2)), "split-K result differs between calls"
    (y,) = _project(rt, torch_dev, [gate], xb, M)
    assert_bf16_close(y, oracle.q4_project(xb, *gate), what="split-K projection")


@pytest.mark.parametrize("knob,q", [("Q", 1), ("Q", 3), ("Q", 8), ("Q", 13), ("Q", 32), ("Q", 45), ("Q", 97),
                                    ("Q", 200), ("SPLITS", 2), ("SPLITS", 3), ("SPLITS", 5), ("SPLITS", 32)])
def test_worker_step_ranges(torch_dev, knob, q):
    # Workers take Q consecutive K steps of the flattened (tile, group) range
    # (QM38_GEMM_Q forces Q; G = 32 here): Q = 32 is whole tiles, Q < 32 cuts
    # every tile into 2 or more pieces, Q > 32 gives ranges that end inside a
    # tile, cross job boundaries and cover whole tiles in between.
    # QM38_GEMM_SPLITS forces S slices per tile instead.  Every choice matches
    # the oracle and repeats bit for bit.
    import qm38
    with tuned(**{"QM38_GEMM_" + knob: q}) as rt:
        rng = np.random.default_rng(700 + q)
        K, M = 2048, 300
        mats = [synth.q4_matrix(rng, 300, K), synth.q4_matrix(rng, 100, K)]
        xb = synth.bf16_normal(rng, (M, K))
        got1 = _project(rt, torch_dev, mats, xb, M)
        got2 = _project(rt, torch_dev, mats, xb, M)
        for (w, s, b), g1, g2 in zip(mats, got1, got2):
            assert_bf16_close(g1, oracle.q4_project(xb, w, s, b), what=f"{knob}={q}")
            assert np.array_equal(g1, g2), f"{knob}={q}: result differs between calls"
        I = 200
        gate, up = synth.q4_matrix(rng, I, K), synth.q4_matrix(rng, I, K)
        dg, du = _upload(torch_dev, *gate), _upload(torch_dev, *up)
        h = empty_bf16((M, I), torch_dev)
        rt.q4_swiglu(qm38.Runtime.job(*dg, I), qm38.Runtime.job(*du, I), to_dev(xb, torch_dev), K, M, h)
        assert_bf16_close(bf16_dev_to_f32(h), oracle.swiglu(oracle.q4_project(xb, *gate), oracle.q4_project(xb, *up)),
                          what=f"swiglu {knob}={q}")


@pytest.mark.parametrize("M", [40, 300])
@pytest.mark.parametrize("knob", [None, ("QM38_GEMM_SPLITS", 3), ("QM38_GEMM_Q", 21)])
def test_mixed_set_in_one_launch(torch_dev, M, knob):
    """qm_q4_project_set with prefill rows: plain projections (256-row tiles)
    and SwiGLU pairs (128 gate + 128 up rows per tile) in one GEMM launch,
    whole tiles, K split into slices, and stream-K ranges that cut tiles of
    both kinds; every output within the bar of the oracle."""
    import qm38
    env = {} if knob is None else {knob[0]: knob[1]}
    with tuned(**env) as rt:
        rng = np.random.default_rng(M + (0 if knob is None else knob[1]))
        K = 1024
        a, g1, u1, b, g2, u2 = (synth.q4_matrix(rng, n, K) for n in (200, 96, 96, 40, 300, 300))
        dev = [_upload(torch_dev, *m) for m in (a, g1, u1, b, g2, u2)]
        ja, jg1, ju1, jb, jg2, ju2 = (qm38.Runtime.job(*d, m[0].shape[0]) for d, m in zip(dev, (a, g1, u1, b, g2, u2)))
        xb = synth.bf16_normal(rng, (M, K))
        outs = [empty_bf16((M, n), torch_dev) for n in (200, 96, 40, 300)]
        rt.q4_project_set([ja, jg1, jb, jg2], [None, ju1, None, ju2], to_dev(xb, torch_dev), K, M, outs)
        assert_bf16_close(bf16_dev_to_f32(outs[0]), oracle.q4_project(xb, *a), what=f"mixed plain M={M}")
        assert_bf16_close(bf16_dev_to_f32(outs[2]), oracle.q4_project(xb, *b), what=f"mixed plain 2 M={M}")
        for o, g, u in ((outs[1], g1, u1), (outs[3], g2, u2)):
            h_ref = oracle.swiglu(oracle.q4_project(xb, *g), oracle.q4_project(xb, *u))
            assert_bf16_close(bf16_dev_to_f32(o), h_ref, what=f"mixed pair M={M} rows {g[0].shape[0]}")
