"""CPU checks that pin the oracle (oracle/) before it is trusted as the GPU
parity checker.  Each test states what fixes the expected answer: the
reference's own known-answer tests (tests/golden/reference_kats.json, values
from /root/reference/src/metal_runtime.rs and src/paged_kv.rs), closed forms,
invariants, or an independent formulation (dequantise-then-GEMM, softmax in
numpy, the DeltaNet recurrence in matrix form).
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest

import oracle
from qm38 import synth

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())
FLT_MIN = np.float32(np.finfo(np.float32).tiny)


# ---------------------------------------------------------------------------
# a0: bf16
# ---------------------------------------------------------------------------
def test_bf16_round_trip_every_finite_value():
    L = oracle.lib()
    bits = np.arange(1 << 16, dtype=np.uint32)
    finite = (bits & 0x7F80) != 0x7F80
    for b in bits[finite][::7]:
        f = L.qo_bf16_to_f32(int(b))
        assert np.float32(f).view(np.uint32) == (int(b) << 16)
        assert L.qo_f32_to_bf16(f) == b


def test_bf16_rounds_half_to_even():
    L = oracle.lib()
    # 1 + 2^-8 is halfway between bf16 1.0 (0x3F80) and 0x3F81: ties to even.
    assert L.qo_f32_to_bf16(np.uint32(0x3F808000).view(np.float32)) == 0x3F80
    assert L.qo_f32_to_bf16(np.uint32(0x3F818000).view(np.float32)) == 0x3F82
    assert L.qo_f32_to_bf16(np.uint32(0x3F808001).view(np.float32)) == 0x3F81
    assert L.qo_f32_to_bf16(np.uint32(0xBF808000).view(np.float32)) == 0xBF80
    # the numpy helper used to build test inputs agrees with the oracle
    rng = np.random.default_rng(0)
    v = (rng.standard_normal(2000) * 10.0 ** rng.integers(-8, 8, 2000)).astype(np.float32)
    assert all(int(synth.f32_to_bf16(np.array([x]))[0]) == L.qo_f32_to_bf16(float(x)) for x in v)


# ---------------------------------------------------------------------------
# a1-a5: Q4 projection
# ---------------------------------------------------------------------------
def _dequant_gemm(xb, packed, s, b):
    """Independent form: dequantise every weight, then one float64 GEMM."""
    q = synth.unpack_q4(packed).astype(np.float64)
    N, K = q.shape
    sf = np.repeat(synth.bf16_to_f32(s).astype(np.float64), 64, axis=1)
    bf = np.repeat(synth.bf16_to_f32(b).astype(np.float64), 64, axis=1)
    W = q * sf + bf
    return synth.bf16_to_f32(xb).astype(np.float64) @ W.T


def test_q4_reference_vectors_k128_n5():
    kat = KATS["q4_k128_n5"]
    K, N = kat["K"], kat["N"]
    x = np.array([((i % 17) - 8) * 0.125 for i in range(K)], np.float32)
    q = np.array([(i * 7 + 3) % 16 for i in range(N * K)], np.uint8).reshape(N, K)
    sc, bc = kat["scales_cycle"], kat["biases_cycle"]
    s = synth.f32_to_bf16(np.array([sc[i % 6] for i in range(N * 2)], np.float32)).reshape(N, 2)
    b = synth.f32_to_bf16(np.array([bc[i % 6] for i in range(N * 2)], np.float32)).reshape(N, 2)
    xb = synth.f32_to_bf16(x)[None]
    packed = synth.pack_q4(q)
    got = oracle.q4_project(xb, packed, s, b)
    # independent scalar evaluation of the reference's CPU formula
    exp = np.zeros((1, N))
    for n in range(N):
        for g in range(K // 64):
            sv, bv = float(synth.bf16_to_f32(s[n, g])), float(synth.bf16_to_f32(b[n, g]))
            for i in range(64 * g, 64 * g + 64):
                exp[0, n] += (sv * q[n, i] + bv) * float(x[i])
    assert np.max(np.abs(got - exp)) < 1e-6  # every value here is exact in binary
    assert np.max(np.abs(got - exp)) < kat["abs_tolerance"]
    np.testing.assert_allclose(got, _dequant_gemm(xb, packed, s, b), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("M,N,K", [(1, 7, 64), (3, 40, 256), (5, 33, 640)])
def test_q4_matches_dequantised_gemm(M, N, K):
    rng = np.random.default_rng(M * 100 + N + K)
    packed, s, b = synth.q4_matrix(rng, N, K)
    xb = synth.bf16_normal(rng, (M, K))
    ref = _dequant_gemm(xb, packed, s, b)
    got = oracle.q4_project(xb, packed, s, b)
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-6 * np.max(np.abs(ref)))
    got32 = oracle.q4_project(xb, packed, s, b, fp32=True)
    assert np.max(np.abs(got32 - ref)) <= 1e-4 * np.max(np.abs(ref))


def test_q4_identity_and_constant_nibbles():
    rng = np.random.default_rng(1)
    N, K, M = 16, 256, 4
    s = synth.f32_to_bf16(rng.uniform(0.005, 0.02, (N, K // 64)).astype(np.float32))
    xb = synth.bf16_normal(rng, (M, K))
    # q = 8, b = -8 s: every weight is exactly zero
    b = synth.f32_to_bf16(-8 * synth.bf16_to_f32(s))
    assert np.all(oracle.q4_project(xb, np.full((N, K // 8), 0x88888888, np.uint32), s, b) == 0.0)
    # q = c: y = sum_g (s c + b) sum_{i in g} x
    c = 13
    b = synth.f32_to_bf16(rng.normal(0, 0.05, (N, K // 64)).astype(np.float32))
    got = oracle.q4_project(xb, np.full((N, K // 8), int("0x" + "d" * 8, 16), np.uint32), s, b)
    xs = synth.bf16_to_f32(xb).astype(np.float64).reshape(M, -1, 64).sum(-1)
    exp = xs @ (synth.bf16_to_f32(s).astype(np.float64) * c + synth.bf16_to_f32(b)).T
    np.testing.assert_allclose(got, exp, rtol=1e-6, atol=1e-7)


def test_swiglu():
    g = np.array([0.0, 1.0, -1.0, 30.0, -30.0, 2.5], np.float32)
    u = np.array([3.0, 2.0, 2.0, 1.0, 1.0, -1.0], np.float32)
    h = oracle.swiglu(g, u)
    assert h[0] == 0.0 and abs(h[3] - 30.0) < 1e-5 and abs(h[4]) < 1e-10
    exp = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    np.testing.assert_allclose(h, exp, rtol=1e-6)


# ---------------------------------------------------------------------------
# a6: Q8 quantisation
# ---------------------------------------------------------------------------
def test_q8_reference_kat():
    q, s = oracle.q8_quantize(np.array([2.0, -1.0], np.float32))
    assert list(q) == KATS["q8_attention_single_token"]["expected_value_q8"]
    assert s == np.float32(2.0) / np.float32(127.0)


def test_q8_rounds_half_away_from_zero_and_floors_scale():
    q, s = oracle.q8_quantize(np.array([127.0, 2.5, -2.5, 1.5, 0.5, -0.5, 0.49], np.float32))
    assert s == np.float32(1.0)
    assert list(q) == [127, 3, -3, 2, 1, -1, 0]
    q, s = oracle.q8_quantize(np.zeros(8, np.float32))
    assert s == FLT_MIN and not q.any()


def test_q8_invariants_random_rows():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((500, 128)) * rng.uniform(1e-3, 1e3, (500, 1))).astype(np.float32)
    q, s = oracle.q8_quantize_rows(x)
    assert np.all(np.abs(q.astype(np.int32)).max(1) == 127)
    r = x / s[:, None]
    assert np.all(np.abs(r - q) <= 0.5 + 1e-6)
    np.testing.assert_array_equal(s, np.maximum(np.abs(x).max(1) / np.float32(127), FLT_MIN))


# ---------------------------------------------------------------------------
# a7: attention
# ---------------------------------------------------------------------------
def _attention_numpy(q, gate, kq, ks, vq, vs, start):
    rows, H, d = q.shape
    T, KVH, _ = kq.shape
    out = np.zeros((rows, H, d))
    for r in range(rows):
        vis = min(start + r + 1, T)
        for h in range(H):
            kv = h * KVH // H
            K = kq[:vis, kv].astype(np.float64) * ks[:vis, kv, None]
            V = vq[:vis, kv].astype(np.float64) * vs[:vis, kv, None]
            sc = K @ q[r, h].astype(np.float64) / math.sqrt(d)
            p = np.exp(sc - sc.max())
            o = (p / p.sum()) @ V
            if gate is not None:
                o = o / (1 + np.exp(-gate[r, h].astype(np.float64)))
            out[r, h] = o
    return out


def test_attention_reference_kat():
    kat = KATS["q8_attention_single_token"]
    kq, ks = oracle.q8_quantize_rows(np.array([[kat["key"]]], np.float32))
    vq, vs = oracle.q8_quantize_rows(np.array([[kat["value"]]], np.float32))
    o = oracle.attention(np.array([[kat["query"]]], np.float32), np.array([[kat["gate"]]], np.float32),
                         kq, ks, vq, vs, 0)[0, 0]
    for got, exp, tol in zip(o, kat["expected"], kat["tolerance"]):
        assert abs(got - exp) < tol
    assert abs(o[1] - (-64 * 2 / 127) * 0.5) < 1e-6  # one token: softmax is the identity


def test_attention_reference_prefill_equals_steps():
    kat = KATS["q8_prefill_matches_steps"]
    q = np.array(kat["queries"], np.float32).reshape(3, 2, 2)
    g = np.array(kat["gates"], np.float32).reshape(3, 2, 2)
    kq, ks = oracle.q8_quantize_rows(np.array(kat["keys"], np.float32).reshape(3, 1, 2))
    vq, vs = oracle.q8_quantize_rows(np.array(kat["values"], np.float32).reshape(3, 1, 2))
    pre = oracle.attention(q, g, kq, ks, vq, vs, 0)
    for t in range(3):
        step = oracle.attention(q[t:t + 1], g[t:t + 1], kq[:t + 1], ks[:t + 1], vq[:t + 1], vs[:t + 1], t)
        np.testing.assert_allclose(pre[t:t + 1], step, rtol=0, atol=1e-7)
    np.testing.assert_allclose(pre, _attention_numpy(q, g, kq, ks, vq, vs, 0), atol=1e-6)


def test_attention_closed_forms_and_numpy():
    rng = np.random.default_rng(3)
    T, KVH, H, d = 37, 2, 6, 64
    k = rng.standard_normal((T, KVH, d)).astype(np.float32)
    v = rng.standard_normal((T, KVH, d)).astype(np.float32)
    kq, ks = oracle.q8_quantize_rows(k)
    vq, vs = oracle.q8_quantize_rows(v)
    q = rng.standard_normal((4, H, d)).astype(np.float32)
    g = rng.standard_normal((4, H, d)).astype(np.float32)
    got = oracle.attention(q, g, kq, ks, vq, vs, 20)
    np.testing.assert_allclose(got, _attention_numpy(q, g, kq, ks, vq, vs, 20), rtol=1e-5, atol=1e-6)
    # identical keys: uniform softmax, output = mean of the visible dequantised V
    kq_u = np.repeat(kq[:1], T, axis=0)
    ks_u = np.repeat(ks[:1], T, axis=0)
    o = oracle.attention(q[:1], None, kq_u, ks_u, vq, vs, T - 1)[0]
    for h in range(H):
        kv = h * KVH // H
        exp = (vq[:, kv].astype(np.float64) * vs[:, kv, None]).mean(0)
        np.testing.assert_allclose(o[h], exp, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------------------
# a8-a10: DeltaNet
# ---------------------------------------------------------------------------
def _dn_numpy(cfg, conv_w, a_log, dt_bias, norm, qkv, z, b, a, eps, hist, S):
    """The recurrence in matrix form, float64 (independent of the oracle's loops)."""
    KH, VH, dk, dv, ks = cfg
    ke = KH * dk
    hist = np.array(hist, np.float64).reshape(qkv.shape[1], ks - 1)
    S = np.array(S, np.float64)
    outs = []
    for t in range(qkv.shape[0]):
        window = np.concatenate([hist, qkv[t].astype(np.float64)[:, None]], axis=1)
        pre = (window * conv_w.astype(np.float64)).sum(1)
        c = pre / (1 + np.exp(-pre))
        hist = window[:, 1:]
        qh = c[:ke].reshape(KH, dk)
        kh = c[ke:2 * ke].reshape(KH, dk)
        qh = qh / np.sqrt((qh ** 2).mean(1, keepdims=True) + eps) / dk
        kh = kh / np.sqrt((kh ** 2).mean(1, keepdims=True) + eps) / np.sqrt(dk)
        v = c[2 * ke:].reshape(VH, dv)
        o = np.zeros((VH, dv))
        for h in range(VH):
            kk, qq = kh[h // (VH // KH)], qh[h // (VH // KH)]
            x = a[t, h] + dt_bias[h]
            sp = x if x > 20 else (math.exp(x) if x < -20 else math.log1p(math.exp(x)))
            g = math.exp(-math.exp(a_log[h]) * sp)
            beta = 1 / (1 + math.exp(-b[t, h]))
            S[h] *= g
            S[h] += np.outer(beta * (v[h] - S[h] @ kk), kk)
            o[h] = S[h] @ qq
        zz = z[t].reshape(VH, dv).astype(np.float64)
        o = o / np.sqrt((o ** 2).mean(1, keepdims=True) + eps) * norm * (zz / (1 + np.exp(-zz)))
        outs.append(o.reshape(-1))
    return np.array(outs), hist, S


def _cfgd(cfg):
    return dict(zip(("key_heads", "value_heads", "key_head_dim", "value_head_dim", "conv_kernel_size"), cfg))


def test_deltanet_reference_vectors_match_matrix_form():
    kat = KATS["deltanet_prefill_matches_steps"]
    cfg = kat["config"]
    conv = np.array(kat["conv_weight"], np.float32).reshape(6, 2)
    args = [np.array(kat[k], np.float32) for k in ("a_log", "dt_bias", "norm")]
    qkv = np.array(kat["qkv"], np.float32).reshape(3, 6)
    z = np.array(kat["z"], np.float32).reshape(3, 2)
    b = np.array(kat["b"], np.float32).reshape(3, 1)
    a = np.array(kat["a"], np.float32).reshape(3, 1)
    hist0, S0 = np.zeros((6, 1)), np.zeros((1, 2, 2))
    for f64 in (False, True):
        out, hist, S = oracle.deltanet_prefill(_cfgd(cfg), conv, *args, qkv, z, b, a, kat["epsilon"], hist0, S0,
                                               f64=f64)
        ref, h_ref, S_ref = _dn_numpy(cfg, conv, *args, qkv, z, b, a, kat["epsilon"], hist0, S0)
        np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(S, S_ref, rtol=1e-5, atol=1e-7)
        np.testing.assert_array_equal(np.asarray(hist).reshape(6, 1), qkv[-1:].T)
        # steps == prefill
        hs, Ss = hist0, S0
        outs = []
        for t in range(3):
            o, hs, Ss = oracle.deltanet_prefill(_cfgd(cfg), conv, *args, qkv[t:t + 1], z[t:t + 1], b[t:t + 1],
                                                a[t:t + 1], kat["epsilon"], hs, Ss, f64=f64)
            outs.append(o[0])
        np.testing.assert_array_equal(np.array(outs), out)


def test_deltanet_scalar_kat_and_precision():
    kat = KATS["deltanet_scalar_recurrence"]
    cfg = kat["config"]
    args = [np.array(kat[k], np.float32) for k in ("a_log", "dt_bias", "norm")]
    qkv = np.array([kat["qkv"]], np.float32)
    z, b, a = (np.array([kat[k]], np.float32) for k in ("z", "b", "a"))
    conv = np.ones((6, 1), np.float32)
    o32, _, _ = oracle.deltanet_prefill(_cfgd(cfg), conv, *args, qkv, z, b, a, kat["epsilon"], np.zeros(0),
                                        np.zeros((1, 2, 2)))
    ref, _, _ = _dn_numpy(cfg, conv, *args, qkv, z, b, a, kat["epsilon"], np.zeros((6, 0)), np.zeros((1, 2, 2)))
    assert np.max(np.abs(o32 - ref)) < kat["tolerance"]
    np.testing.assert_allclose(o32, ref, rtol=1e-5, atol=1e-6)


def test_deltanet_f32_matches_f64_at_model_head_size():
    rng = np.random.default_rng(5)
    cfg = (2, 4, 128, 128, 4)
    ch = 2 * 2 * 128 + 4 * 128
    conv = (rng.standard_normal((ch, 4)) * 0.5).astype(np.float32)
    a_log, dt_bias = np.zeros(4, np.float32), np.zeros(4, np.float32)
    norm = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    M = 20
    qkv = rng.standard_normal((M, ch)).astype(np.float32)
    z = rng.standard_normal((M, 512)).astype(np.float32)
    b = rng.standard_normal((M, 4)).astype(np.float32)
    a = rng.standard_normal((M, 4)).astype(np.float32)
    h0, S0 = np.zeros((ch, 3)), np.zeros((4, 128, 128))
    o32, _, S32 = oracle.deltanet_prefill(_cfgd(cfg), conv, a_log, dt_bias, norm, qkv, z, b, a, 1e-6, h0, S0)
    o64, _, S64 = oracle.deltanet_prefill(_cfgd(cfg), conv, a_log, dt_bias, norm, qkv, z, b, a, 1e-6, h0, S0,
                                          f64=True)
    assert np.max(np.abs(o32 - o64)) <= 1e-5 * np.max(np.abs(o64))
    assert np.max(np.abs(S32 - S64)) <= 1e-5 * np.max(np.abs(S64))
    ref, _, S_ref = _dn_numpy(cfg, conv, a_log, dt_bias, norm, qkv[:4], z[:4], b[:4], a[:4], 1e-6, h0, S0)
    o4, _, S4 = oracle.deltanet_prefill(_cfgd(cfg), conv, a_log, dt_bias, norm, qkv[:4], z[:4], b[:4], a[:4], 1e-6,
                                        h0, S0, f64=True)
    np.testing.assert_allclose(o4, ref, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(S4, S_ref, rtol=1e-6, atol=1e-9)


def test_deltanet_closed_forms():
    rng = np.random.default_rng(6)
    cfg = (1, 2, 32, 16, 1)
    ch = 2 * 32 + 2 * 16
    conv = np.ones((ch, 1), np.float32)
    z0 = np.zeros(2, np.float32)
    norm = np.ones(16, np.float32)
    qkv = rng.standard_normal((1, ch)).astype(np.float32)
    z = rng.standard_normal((1, 32)).astype(np.float32)
    a = rng.standard_normal((1, 2)).astype(np.float32)
    S0 = rng.standard_normal((2, 16, 32))
    # beta = 0: S <- g S with g = exp(-softplus(a))
    _, _, S = oracle.deltanet_prefill(_cfgd(cfg), conv, z0, z0, norm, qkv, z, np.full((1, 2), -200, np.float32), a,
                                      1e-6, np.zeros(0), S0, f64=True)
    g = np.exp(-np.log1p(np.exp(a[0].astype(np.float64))))
    np.testing.assert_allclose(S, S0 * g[:, None, None], rtol=1e-12)
    # g = 1, beta = 1, eps = 0: S k^ = v after the update
    _, _, S = oracle.deltanet_prefill(_cfgd(cfg), conv, z0, z0, norm, qkv, z, np.full((1, 2), 200, np.float32),
                                      np.full((1, 2), -200, np.float32), 0.0, np.zeros(0), S0, f64=True)
    c = qkv[0].astype(np.float64) / (1 + np.exp(-qkv[0].astype(np.float64)))
    k = c[32:64] / np.linalg.norm(c[32:64])
    for h in range(2):
        np.testing.assert_allclose(S[h] @ k, c[64 + 16 * h:80 + 16 * h], rtol=1e-9, atol=1e-12)


# ---------------------------------------------------------------------------
# a7c: page table
# ---------------------------------------------------------------------------
def test_page_table_reference_tests():
    # paged_kv.rs:136-163
    t = oracle.LogicalPageTable(262_144, 128)
    assert t.allocated_pages() == 0
    t.append(127)
    assert t.allocated_pages() == 1 and t.page_for_token(0) == 0
    t.append(1)
    assert t.allocated_pages() == 1
    t.append(1)
    assert t.allocated_pages() == 2 and t.page_for_token(128) == 1
    t = oracle.LogicalPageTable(128, 128)
    t.append(128)
    with pytest.raises(oracle.PageTableError):
        t.append(1)


def test_page_table_invariants():
    with pytest.raises(oracle.PageTableError):
        oracle.LogicalPageTable(0, 16)
    t = oracle.LogicalPageTable(1000, 16)
    with pytest.raises(oracle.PageTableError):
        t.append(0)
    rng = np.random.default_rng(8)
    n = 0
    while True:
        k = int(rng.integers(1, 40))
        if n + k > 1000:
            with pytest.raises(oracle.PageTableError):
                t.append(k)
            break
        start, end, first, last = t.append(k)
        assert (start, end, first, last) == (n, n + k, n // 16, (n + k - 1) // 16)
        n += k
        assert t.allocated_pages() == -(-n // 16)
    assert all(t.page_for_token(i) == i // 16 for i in range(n))
    assert t.page_for_token(n) is None


# ---------------------------------------------------------------------------
# Full-attention q/k preparation (RMSNorm + (M-)RoPE + query/gate split)
# ---------------------------------------------------------------------------
# metal_runtime.rs:9370-9420 gqa_gpu_prepare_matches_rms_norm_and_mrope inputs.
PREP_QG = np.array([0.25, -0.5, 0.75, -1.0, 0.1, 0.2, 0.3, 0.4,
                    -0.3, 0.6, -0.9, 1.2, -0.2, -0.1, 0.0, 0.1], np.float32).reshape(1, 2, 8)
PREP_K = np.array([0.5, -0.25, 0.75, -1.0], np.float32).reshape(1, 1, 4)
PREP_QN = np.array([0.9, 1.0, 1.1, 1.2], np.float32)
PREP_KN = np.array([1.2, 1.1, 1.0, 0.9], np.float32)
PREP_POS = np.array([[7], [11], [13]], np.uint32)


def test_attn_prepare_reference_kat():
    q, g, k = oracle.attn_prepare(PREP_QG, PREP_K, PREP_QN, PREP_KN, 4, 4, 10000.0, 1e-6, sections=(1, 1),
                                  positions=PREP_POS)
    # Key, by hand: mean x^2 = 0.46875, scale = 1/sqrt(0.468751); pair 0 turns
    # by 7 rad (axis 0), pair 1 by 11/100 rad (frequency 1 -> axis 1 because
    # 1 % 3 == 1 and 1 / 3 < section1).
    s = 1.0 / math.sqrt(0.46875 + 1e-6)
    n = [0.5 * s * 1.2, -0.25 * s * 1.1, 0.75 * s * 1.0, -1.0 * s * 0.9]
    c0, s0, c1, s1 = math.cos(7), math.sin(7), math.cos(0.11), math.sin(0.11)
    want = [n[0] * c0 - n[2] * s0, n[1] * c1 - n[3] * s1, n[2] * c0 + n[0] * s0, n[3] * c1 + n[1] * s1]
    np.testing.assert_allclose(k[0, 0], want, rtol=2e-6, atol=2e-6)
    assert abs(k[0, 0, 0] - (-0.0590059)) < 1e-5 and abs(k[0, 0, 2] - 1.4016113) < 1e-5
    # Gates are the second half of each head, copied.
    np.testing.assert_array_equal(g[0], PREP_QG[0, :, 4:])
    # Heads 0 and 1 of the query are negatives of each other up to the weight:
    # head 1 = -1.2 * head 0, and RMSNorm is scale invariant.
    np.testing.assert_allclose(q[0, 1], -q[0, 0], rtol=1e-5, atol=1e-6)


def test_attn_prepare_invariants():
    rng = np.random.default_rng(5)
    M, H, KVH, hd, rd = 6, 4, 2, 128, 32
    qg = rng.standard_normal((M, H, 2 * hd)).astype(np.float32)
    kin = rng.standard_normal((M, KVH, hd)).astype(np.float32)
    qn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    zero = np.zeros((3, M), np.uint32)
    q0, _, k0 = oracle.attn_prepare(qg, kin, qn, kn, hd, rd, 1e6, 1e-6, positions=zero)
    # Position 0 rotates nothing: plain RMSNorm (rotary_dim 0 gives the same).
    qr, _, kr = oracle.attn_prepare(qg, kin, qn, kn, hd, 0, 1e6, 1e-6, positions=zero)
    np.testing.assert_array_equal(q0, qr)
    np.testing.assert_array_equal(k0, kr)
    x = qg[..., :hd].astype(np.float64)
    ref = x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6) * qn
    np.testing.assert_allclose(q0, ref, rtol=1e-5, atol=1e-6)
    # Rotation preserves each pair's norm and leaves dims >= rotary_dim alone.
    pos = rng.integers(0, 200000, (3, M)).astype(np.uint32)
    q1, _, k1 = oracle.attn_prepare(qg, kin, qn, kn, hd, rd, 1e6, 1e-6, sections=(5, 5), positions=pos)
    h = rd // 2
    for a, b in ((q0, q1), (k0, k1)):
        np.testing.assert_allclose(a[..., :h] ** 2 + a[..., h:rd] ** 2, b[..., :h] ** 2 + b[..., h:rd] ** 2,
                                   rtol=1e-4, atol=1e-6)
        np.testing.assert_array_equal(a[..., rd:], b[..., rd:])
    # Text rows: q(p1) . k(p2) over the rotary part depends only on p1 - p2.
    def dot(p1, p2):
        qa, _, _ = oracle.attn_prepare(qg[:1], kin[:1], qn, kn, hd, rd, 1e4, 1e-6, base=p1)
        _, _, kb = oracle.attn_prepare(qg[:1], kin[:1], qn, kn, hd, rd, 1e4, 1e-6, base=p2)
        return float(np.dot(qa[0, 0, :rd].astype(np.float64), kb[0, 0, :rd]))
    assert abs(dot(9, 4) - dot(1009, 1004)) < 1e-4
    assert abs(dot(9, 4) - dot(10, 4)) > 1e-3  # and it does depend on the offset


def test_attn_prepare_mrope_axis_selection():
    # Frequency i uses axis 1 iff i % 3 == 1 and i / 3 < s1, axis 2 iff
    # i % 3 == 2 and i / 3 < s2 (native.rs:136-148): moving only position 1
    # changes exactly those pairs.
    rng = np.random.default_rng(8)
    hd, rd, s1, s2 = 64, 48, 3, 2
    qg = rng.standard_normal((1, 1, 2 * hd)).astype(np.float32)
    kin = rng.standard_normal((1, 1, hd)).astype(np.float32)
    w = np.ones(hd, np.float32)
    base = np.array([[100], [200], [300]], np.uint32)
    moved = base.copy()
    moved[1, 0] = 777
    _, _, a = oracle.attn_prepare(qg, kin, w, w, hd, rd, 1e4, 1e-6, sections=(s1, s2), positions=base)
    _, _, b = oracle.attn_prepare(qg, kin, w, w, hd, rd, 1e4, 1e-6, sections=(s1, s2), positions=moved)
    h = rd // 2
    changed = {i for i in range(h) if a[0, 0, i] != b[0, 0, i] or a[0, 0, i + h] != b[0, 0, i + h]}
    assert changed == {i for i in range(h) if i % 3 == 1 and i // 3 < s1}
    # Without sections every frequency uses axis 0.
    _, _, c = oracle.attn_prepare(qg, kin, w, w, hd, rd, 1e4, 1e-6, positions=base)
    _, _, d = oracle.attn_prepare(qg, kin, w, w, hd, rd, 1e4, 1e-6, positions=moved)
    np.testing.assert_array_equal(c, d)


# ---- residual add + RMSNorm (qo_residual_rmsnorm; qwen38.metal:4253-4333) --
def test_rmsnorm_known_answers():
    # [3, 4]: mean square 12.5, scale 1/sqrt(12.5); weights [1, 2] as given.
    _, out = oracle.residual_rmsnorm(np.array([[3.0, 4.0]], np.float32), np.array([1.0, 2.0], np.float32), 0.0)
    s = 1 / np.sqrt(12.5)
    np.testing.assert_allclose(out[0], [3 * s, 8 * s], rtol=1e-15)
    # A constant row normalises to its sign times the weights.
    _, out = oracle.residual_rmsnorm(np.full((2, 7), -2.5, np.float32), np.full(7, 0.5, np.float32), 0.0)
    np.testing.assert_allclose(out, np.full((2, 7), -0.5), rtol=1e-15)


def test_rmsnorm_invariants():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 40)).astype(np.float32)
    w = rng.standard_normal(40).astype(np.float32)
    _, a = oracle.residual_rmsnorm(x, w, 0.0)
    _, b = oracle.residual_rmsnorm(4 * x, w, 0.0)  # scale invariance (exact power-of-two scaling)
    np.testing.assert_allclose(a, b, rtol=1e-14)
    # Unit-RMS output with unit weights; zero weights give zero (weights are not 1 + w).
    _, u = oracle.residual_rmsnorm(x, np.ones(40, np.float32), 0.0)
    np.testing.assert_allclose(np.sqrt(np.mean(u ** 2, axis=1)), 1.0, rtol=1e-12)
    _, z = oracle.residual_rmsnorm(x, np.zeros(40, np.float32), 1e-6)
    assert not np.any(z)
    # eps keeps an all-zero row finite.
    _, e = oracle.residual_rmsnorm(np.zeros((1, 8), np.float32), np.ones(8, np.float32), 1e-6)
    assert np.all(e == 0)
    # The residual add is plain fp32 addition, row by row.
    d = rng.standard_normal((3, 40)).astype(np.float32)
    h, r = oracle.residual_rmsnorm(x, w, 1e-6, d)
    np.testing.assert_array_equal(h, x + d)
    _, r2 = oracle.residual_rmsnorm(x + d, w, 1e-6)
    np.testing.assert_array_equal(r, r2)
