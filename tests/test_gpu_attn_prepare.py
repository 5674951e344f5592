"""GPU parity of the full-attention q/k preparation (qm_attn_prepare) against
the CPU oracle: per-head RMSNorm, partial (M-)RoPE and the query/gate split of
qwen38_gqa_prepare_query(_rows) / _key(_rows) (qwen38.metal:4761-5029; CPU
native.rs:4917-4942, 5153-5180).

Ports metal_runtime.rs:9370 gqa_gpu_prepare_matches_rms_norm_and_mrope (its
inputs rounded to bf16, the kernel's input type), plus Qwen3.5 full-attention
shapes with text and M-RoPE positions up to 128K.  Tolerances: query bf16
within 1e-4 of max|ref| beyond the final rounding; key fp32 within 2e-5 of
max|ref|; gate bit-exact (a copy).  Both sides evaluate the rotation angle in
fp64, so the budget covers fp32 rounding and summation order only.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from gpu_util import assert_bf16_close, bf16_dev_to_f32, empty_bf16, from_dev, to_dev
from qm38 import QmError, synth

pytestmark = pytest.mark.gpu


def _rope(hd, rd, theta, sections=None):
    import qm38
    s1, s2 = sections if sections is not None else (0, 0)
    return qm38.RopeConfig(hd, rd, theta, s1, s2, int(sections is not None))


def _run(rt, dev, qg_bits, k_bits, qn, kn, hd, rd, theta, eps, sections=None, positions=None, base=0):
    import torch
    M, H, KVH = qg_bits.shape[0], qg_bits.shape[1], k_bits.shape[1]
    q = empty_bf16((M, H, hd), dev)
    g = empty_bf16((M, H, hd), dev)
    k = torch.full((M, KVH, hd), float("nan"), dtype=torch.float32, device=dev)
    pos = None if positions is None else to_dev(positions.astype(np.uint32), dev)
    rt.attn_prepare(_rope(hd, rd, theta, sections), M, H, KVH, to_dev(qg_bits, dev), to_dev(k_bits, dev),
                    to_dev(qn.astype(np.float32), dev), to_dev(kn.astype(np.float32), dev), eps, q, g, k,
                    positions=pos, position_base=base)
    return bf16_dev_to_f32(q), from_dev(g, np.uint16), from_dev(k)


def _check(rt, dev, qg_bits, k_bits, qn, kn, hd, rd, theta, eps=1e-6, sections=None, positions=None, base=0,
           what=""):
    q, g, k = _run(rt, dev, qg_bits, k_bits, qn, kn, hd, rd, theta, eps, sections, positions, base)
    rq, _, rk = oracle.attn_prepare(synth.bf16_to_f32(qg_bits), synth.bf16_to_f32(k_bits), qn, kn, hd, rd, theta,
                                    eps, sections=sections, positions=positions, base=base)
    assert_bf16_close(q, rq, what=f"{what} query")
    np.testing.assert_array_equal(g, qg_bits[..., hd:], err_msg=f"{what} gate")
    assert np.all(np.isfinite(k)), f"{what}: key not written"
    np.testing.assert_allclose(k, rk, rtol=0, atol=2e-5 * max(np.abs(rk).max(), 1e-30), err_msg=f"{what} key")


def test_reference_fixture(rt, torch_dev):
    # metal_runtime.rs:9370-9420: 2 query heads, 1 KV head, head_dim 4,
    # rotary_dim 4, positions (7, 11, 13), sections (1, 1), theta 1e4.
    qg = np.array([0.25, -0.5, 0.75, -1.0, 0.1, 0.2, 0.3, 0.4,
                   -0.3, 0.6, -0.9, 1.2, -0.2, -0.1, 0.0, 0.1], np.float32).reshape(1, 2, 8)
    k = np.array([0.5, -0.25, 0.75, -1.0], np.float32).reshape(1, 1, 4)
    qn = np.array([0.9, 1.0, 1.1, 1.2], np.float32)
    kn = np.array([1.2, 1.1, 1.0, 0.9], np.float32)
    pos = np.array([[7], [11], [13]], np.uint32)
    _check(rt, torch_dev, synth.f32_to_bf16(qg), synth.f32_to_bf16(k), qn, kn, 4, 4, 10000.0, sections=(1, 1),
           positions=pos, what="fixture")


@pytest.mark.parametrize("M,H,KVH,hd,rd", [(1, 24, 4, 256, 64), (7, 24, 4, 256, 64), (64, 16, 2, 128, 32),
                                           (3, 8, 8, 64, 64), (5, 6, 2, 200, 50), (2, 4, 1, 256, 0)])
@pytest.mark.parametrize("mode", ["text", "mrope"])
def test_matches_oracle(rt, torch_dev, M, H, KVH, hd, rd, mode):
    rng = np.random.default_rng(M * 131 + H * 7 + hd + rd + (mode == "mrope"))
    qg = synth.bf16_normal(rng, (M, H, 2 * hd))
    k = synth.bf16_normal(rng, (M, KVH, hd))
    qn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    if mode == "text":
        _check(rt, torch_dev, qg, k, qn, kn, hd, rd, 1e7, base=int(rng.integers(0, 131072)), what="text")
    else:
        pos = rng.integers(0, 131072, (3, M)).astype(np.uint32)
        _check(rt, torch_dev, qg, k, qn, kn, hd, rd, 1e7, sections=(11, 10), positions=pos, what="mrope")


def test_prepared_rows_feed_decode_attention(rt, torch_dev):
    # prepare -> qm_attn_decode: the attention output equals the oracle's
    # attention over the oracle-prepared q/k (KV quantised by the same rule).
    rng = np.random.default_rng(21)
    H, KVH, hd, rd, T = 8, 2, 128, 32, 40
    cache = rt.create_q8_kv_state(KVH, hd, T + 8)
    qn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    keys, vals = [], []
    for t in range(T):
        qg = synth.bf16_normal(rng, (1, H, 2 * hd))
        kb = synth.bf16_normal(rng, (1, KVH, hd))
        q, g, k = _run(rt, torch_dev, qg, kb, qn, kn, hd, rd, 1e7, 1e-6, base=t)
        v = rng.standard_normal((1, KVH, hd)).astype(np.float32)
        o = empty_bf16((1, H, hd), torch_dev)
        rt.gqa_attention_q8([cache], to_dev(synth.f32_to_bf16(q), torch_dev), to_dev(g, torch_dev),
                            to_dev(k, torch_dev), to_dev(v, torch_dev), H, o)
        keys.append(k[0])
        vals.append(v[0])
    kq, ks = oracle.q8_quantize_rows(np.stack(keys))
    vq, vs = oracle.q8_quantize_rows(np.stack(vals))
    ref = oracle.attention(q, synth.bf16_to_f32(g), kq, ks, vq, vs, T - 1)
    assert_bf16_close(bf16_dev_to_f32(o), ref, what="decode after prepare")
    cache.close()


def test_rejects_bad_shapes(rt, torch_dev):
    import torch
    qg = torch.zeros((1, 2, 8), dtype=torch.int16, device=torch_dev)
    k = torch.zeros((1, 1, 4), dtype=torch.int16, device=torch_dev)
    w = torch.ones(4, dtype=torch.float32, device=torch_dev)
    q = torch.zeros((1, 2, 4), dtype=torch.int16, device=torch_dev)
    ko = torch.zeros((1, 1, 4), dtype=torch.float32, device=torch_dev)
    for rope, rows in ((_rope(4, 3, 1e4), 1), (_rope(4, 6, 1e4), 1), (_rope(300, 4, 1e4), 1),
                       (_rope(4, 4, 0.0), 1), (_rope(4, 4, 1e4), 0)):
        with pytest.raises(QmError):
            rt.attn_prepare(rope, rows, 2, 1, qg, k, w, w, 1e-6, q, q, ko)
    with pytest.raises(QmError):
        rt.attn_prepare(_rope(4, 4, 1e4), 1, 2, 1, qg, k, w, w, 1e-6, q, None, ko)
