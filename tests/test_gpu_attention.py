"""GPU parity of the paged Q8-KV GQA attention against the CPU oracle.

Ports metal_runtime.rs tests q8_gqa_attention_keeps_kv_on_the_gpu (:11587),
q8_gqa_prefill_matches_steps_and_keeps_kv_state (:11608) and
q8_gqa_prefill_matches_steps_when_kv_capacity_grows (:11683), plus seeded
cases at the model's shapes (head_dim 256, GQA groups up to 16, ragged
batches, split-K decode up to 32K tokens).

The reference tests use head_dim 2; this build's kernels take head_dim 64,
128 or 256.  The reference vectors are embedded by zero-padding q, k and v
to 64 and scaling q by sqrt(64/2): zero lanes change neither the absmax of
a row (so the int8 bytes and scales are the reference's) nor any dot
product, and the scaling keeps q.k/sqrt(d) identical.

Bars: quantised cache bytes and scales bit-exact against the oracle's
quantiser; page tables identical to LogicalPageTable; outputs (bf16) within
2e-3 of max|ref| beyond bf16 rounding, against an fp64-accumulated oracle
fed the same bf16 q and gate.
"""
from __future__ import annotations

import math
import os

import numpy as np
import pytest

import oracle
from gpu_util import assert_bf16_close, bf16_dev_to_f32, empty_bf16, to_dev
from qm38 import QmError, synth

pytestmark = pytest.mark.gpu


class Mirror:
    """Host copy of one sequence's appended fp32 K/V rows."""

    def __init__(self, kvh, d):
        self.k = np.zeros((0, kvh, d), np.float32)
        self.v = np.zeros((0, kvh, d), np.float32)

    def append(self, k, v):
        self.k = np.concatenate([self.k, k.reshape(-1, *self.k.shape[1:])])
        self.v = np.concatenate([self.v, v.reshape(-1, *self.v.shape[1:])])

    def truncate(self, n):
        self.k, self.v = self.k[:n], self.v[:n]

    def quantised(self):
        kq, ks = oracle.q8_quantize_rows(self.k)
        vq, vs = oracle.q8_quantize_rows(self.v)
        return kq, ks, vq, vs

    def reference(self, q, gate, start):
        kq, ks, vq, vs = self.quantised()
        return oracle.attention(q, gate, kq, ks, vq, vs, start)


def _bf16(a):
    bits = synth.f32_to_bf16(np.asarray(a, np.float32))
    return bits, synth.bf16_to_f32(bits)


def _decode(rt, dev, caches, q_bits, g_bits, k, v, H):
    B, _, D = q_bits.shape
    o = empty_bf16((B, H, D), dev)
    rt.gqa_attention_q8(caches, to_dev(q_bits, dev), None if g_bits is None else to_dev(g_bits, dev),
                        to_dev(k, dev), to_dev(v, dev), H, o)
    return bf16_dev_to_f32(o)


def _prefill(rt, dev, cache, q_bits, g_bits, k, v, H):
    M, _, D = q_bits.shape
    o = empty_bf16((M, H, D), dev)
    rt.gqa_attention_q8_prefill(cache, to_dev(q_bits, dev), None if g_bits is None else to_dev(g_bits, dev),
                                to_dev(k, dev), to_dev(v, dev), H, M, o)
    return bf16_dev_to_f32(o)


def _check_cache(cache, mirror):
    keys, values, ks, vs = cache.read()
    kq, kss, vq, vss = mirror.quantised()
    assert np.array_equal(keys, kq), "K bytes differ from the oracle quantiser"
    assert np.array_equal(values, vq), "V bytes differ from the oracle quantiser"
    assert np.array_equal(ks.view(np.uint32), kss.view(np.uint32)), "K scales differ"
    assert np.array_equal(vs.view(np.uint32), vss.view(np.uint32)), "V scales differ"


# ---------------------------------------------------------------------------
# Reference known-answer tests (head_dim 2 embedded in 64)
# ---------------------------------------------------------------------------
PAD_D = 64
QSCALE = math.sqrt(PAD_D / 2)


def _pad(a, heads):
    a = np.asarray(a, np.float32).reshape(-1, heads, 2)
    out = np.zeros((a.shape[0], heads, PAD_D), np.float32)
    out[..., :2] = a
    return out


def test_reference_kat_single_token(rt, torch_dev):
    # metal_runtime.rs:11587-11605
    cache = rt.create_q8_kv_state(1, PAD_D, 64)
    q_bits, _ = _bf16(_pad([1.0, 0.0], 1) * QSCALE)
    g_bits, _ = _bf16(_pad([0.0, 0.0], 1))
    out = _decode(rt, torch_dev, [cache], q_bits, g_bits, _pad([1.0, 0.0], 1), _pad([2.0, -1.0], 1), 1)
    assert cache.sequence_length == 1
    assert abs(out[0, 0, 0] - 1.0) < 0.001, out[0, 0, :2]
    assert abs(out[0, 0, 1] + 0.5) < 0.005, out[0, 0, :2]
    # zero-padded dimensions: only the rounding residual of the fp16 hi+lo P'V split remains
    assert np.max(np.abs(out[0, 0, 2:])) < 1e-3
    keys, values, ks, vs = cache.read()
    assert list(values[0, 0, :2]) == [127, -64] and ks[0, 0] == np.float32(1.0) / np.float32(127.0)
    assert vs[0, 0] == np.float32(2.0) / np.float32(127.0)


def test_reference_kat_prefill_matches_steps(rt, torch_dev):
    # metal_runtime.rs:11608-11682 (H=2, KVH=1)
    queries = [1.0, 0.0, 0.25, -0.5, 0.5, 0.5, -0.75, 0.25, -0.2, 0.8, 0.6, -0.4]
    gates = [0.0, 0.0, 0.1, -0.1, -0.2, 0.2, 0.0, 0.0, 0.3, -0.3, 0.15, 0.05]
    keys = [1.0, 0.0, 0.4, 0.9, -0.7, 0.2]
    values = [2.0, -1.0, 0.75, 1.25, -0.5, 0.4]
    q_bits, q_f = _bf16(_pad(queries, 2) * QSCALE)
    g_bits, g_f = _bf16(_pad(gates, 2))
    k, v = _pad(keys, 1), _pad(values, 1)
    step = rt.create_q8_kv_state(1, PAD_D, 64)
    pre = rt.create_q8_kv_state(1, PAD_D, 64)
    expected = np.concatenate([_decode(rt, torch_dev, [step], q_bits[t:t + 1], g_bits[t:t + 1], k[t], v[t], 2)
                               for t in range(3)])
    actual = _prefill(rt, torch_dev, pre, q_bits, g_bits, k, v, 2)
    assert pre.sequence_length == 3
    assert np.max(np.abs(actual - expected)) < 0.005
    mirror = Mirror(1, PAD_D)
    mirror.append(k, v)
    assert_bf16_close(actual, mirror.reference(q_f, g_f, 0), what="kat prefill")
    _check_cache(pre, mirror)
    _check_cache(step, mirror)

    nq_bits, nq_f = _bf16(_pad([0.9, -0.1, -0.3, 0.7], 2) * QSCALE)
    ng_bits, ng_f = _bf16(_pad([0.05, -0.05, 0.2, -0.2], 2))
    nk, nv = _pad([0.2, -0.6], 1), _pad([1.1, -0.8], 1)
    e_next = _decode(rt, torch_dev, [step], nq_bits, ng_bits, nk, nv, 2)
    a_next = _decode(rt, torch_dev, [pre], nq_bits, ng_bits, nk, nv, 2)
    assert np.max(np.abs(a_next - e_next)) < 0.005
    mirror.append(nk, nv)
    assert_bf16_close(a_next, mirror.reference(nq_f, ng_f, 3), what="kat next")


def test_reference_kat_capacity_grows(rt, torch_dev):
    # metal_runtime.rs:11683-11803: 16 steps vs one 16-row prefill, reserve 3,
    # then 3 steps vs a 3-row prefill; cache bytes identical throughout.
    def row(t):
        return ([0.15 + t * 0.01, -0.4 + t * 0.02, 0.2 - t * 0.01, 0.3 + t * 0.015],
                [0.05 - t * 0.01, -0.1 + t * 0.005, 0.02 + t * 0.01, -0.03],
                [0.5 + t * 0.01, -0.7 + t * 0.005], [0.8 - t * 0.02, -0.2 + t * 0.01])

    rows = [row(t) for t in range(19)]
    q_bits, q_f = _bf16(_pad([x for r in rows for x in r[0]], 2) * QSCALE)
    g_bits, g_f = _bf16(_pad([x for r in rows for x in r[1]], 2))
    k = _pad([x for r in rows for x in r[2]], 1)
    v = _pad([x for r in rows for x in r[3]], 1)
    step = rt.create_q8_kv_state(1, PAD_D, 19)
    pre = rt.create_q8_kv_state(1, PAD_D, 19)
    for t in range(16):
        _decode(rt, torch_dev, [step], q_bits[t:t + 1], g_bits[t:t + 1], k[t], v[t], 2)
    _prefill(rt, torch_dev, pre, q_bits[:16], g_bits[:16], k[:16], v[:16], 2)
    mirror = Mirror(1, PAD_D)
    mirror.append(k[:16], v[:16])
    _check_cache(step, mirror)
    _check_cache(pre, mirror)
    step.reserve(3)
    pre.reserve(3)
    assert step.allocated_pages == pre.allocated_pages == 2
    _check_cache(pre, mirror)
    expected = np.concatenate([_decode(rt, torch_dev, [step], q_bits[t:t + 1], g_bits[t:t + 1], k[t], v[t], 2)
                               for t in range(16, 19)])
    actual = _prefill(rt, torch_dev, pre, q_bits[16:], g_bits[16:], k[16:], v[16:], 2)
    assert step.sequence_length == pre.sequence_length == 19
    mirror.append(k[16:], v[16:])
    _check_cache(step, mirror)
    _check_cache(pre, mirror)
    assert np.max(np.abs(actual - expected)) < 0.005
    assert_bf16_close(actual, mirror.reference(q_f[16:], g_f[16:], 16), what="grown prefill")
    with pytest.raises(QmError, match="CAPACITY_EXCEEDED"):
        _decode(rt, torch_dev, [step], q_bits[:1], g_bits[:1], k[0], v[0], 2)
    assert step.sequence_length == 19


# ---------------------------------------------------------------------------
# Seeded parity at model shapes
# ---------------------------------------------------------------------------
def _rand_qkv(rng, n, H, KVH, D, gate=True):
    q_bits, q_f = _bf16(rng.standard_normal((n, H, D)).astype(np.float32))
    g_bits, g_f = _bf16(rng.standard_normal((n, H, D)).astype(np.float32)) if gate else (None, None)
    k = (rng.standard_normal((n, KVH, D)) * 1.5).astype(np.float32)
    v = rng.standard_normal((n, KVH, D)).astype(np.float32)
    return q_bits, q_f, g_bits, g_f, k, v


def _fill(rt, dev, cache, mirror, rng, n, H, KVH, D):
    """Prefill n random rows (no output check)."""
    if n == 0:
        return
    q_bits, _, _, _, k, v = _rand_qkv(rng, n, H, KVH, D, gate=False)
    _prefill(rt, dev, cache, q_bits, None, k, v, H)
    mirror.append(k, v)


@pytest.mark.parametrize("D,H,KVH", [(256, 24, 4), (128, 64, 8), (128, 16, 2), (64, 8, 8), (256, 16, 1),
                                      (128, 32, 4)])
@pytest.mark.parametrize("pps", [0, 1])
def test_decode_ragged_batch(rt, torch_dev, D, H, KVH, pps):
    rng = np.random.default_rng(D * 7 + H * 3 + KVH + pps)
    lens = [0, 15, 16, 17, 100, 333]
    caches = [rt.create_q8_kv_state(KVH, D, 512) for _ in lens]
    mirrors = [Mirror(KVH, D) for _ in lens]
    for c, m, n in zip(caches, mirrors, lens):
        _fill(rt, torch_dev, c, m, rng, n, H, KVH, D)
    if pps:
        os.environ["QM38_ATTN_PPS"] = str(pps)
    try:
        for it in range(2):
            q_bits, q_f, g_bits, g_f, k, v = _rand_qkv(rng, len(lens), H, KVH, D, gate=(it == 0))
            got = _decode(rt, torch_dev, caches, q_bits, g_bits, k, v, H)
            for b, (c, m) in enumerate(zip(caches, mirrors)):
                m.append(k[b], v[b])
                assert c.sequence_length == m.k.shape[0]
                ref = m.reference(q_f[b:b + 1], None if g_f is None else g_f[b:b + 1], m.k.shape[0] - 1)
                assert_bf16_close(got[b:b + 1], ref, what=f"seq {b} len {m.k.shape[0]} it {it}")
    finally:
        os.environ.pop("QM38_ATTN_PPS", None)
    for c, m in zip(caches, mirrors):
        _check_cache(c, m)


@pytest.mark.parametrize("D,H,KVH", [(128, 64, 8), (64, 8, 8)])
def test_decode_long_split_page_ids(rt, torch_dev, D, H, KVH):
    """Splits of 320 pages give each wave 80 pages: the first 64 ids come from
    the per-wave id vector, the rest (including the page this step
    materialises, page 620 = wave 0's 76th page of split 1) from scalar loads."""
    rng = np.random.default_rng(D + H)
    n = 620 * 16
    cache = rt.create_q8_kv_state(KVH, D, n + 64)
    mirror = Mirror(KVH, D)
    _fill(rt, torch_dev, cache, mirror, rng, n, H, KVH, D)
    os.environ["QM38_ATTN_PPS"] = "320"
    try:
        for it in range(2):
            q_bits, q_f, g_bits, g_f, k, v = _rand_qkv(rng, 1, H, KVH, D, gate=(it == 1))
            got = _decode(rt, torch_dev, [cache], q_bits, g_bits, k, v, H)
            mirror.append(k[0], v[0])
            ref = mirror.reference(q_f, g_f, mirror.k.shape[0] - 1)
            assert_bf16_close(got, ref, what=f"len {mirror.k.shape[0]} it {it}")
    finally:
        os.environ.pop("QM38_ATTN_PPS", None)
    _check_cache(cache, mirror)


@pytest.mark.parametrize("D,H,KVH", [(256, 24, 4), (128, 64, 8), (128, 16, 2), (64, 4, 4), (256, 16, 1)])
@pytest.mark.parametrize("start,M", [(0, 1), (0, 5), (0, 16), (0, 77), (13, 40), (32, 33), (200, 300)])
def test_prefill_matches_oracle(rt, torch_dev, D, H, KVH, start, M):
    rng = np.random.default_rng(start * 1000 + M + D + H)
    cache = rt.create_q8_kv_state(KVH, D, start + M + 8)
    mirror = Mirror(KVH, D)
    _fill(rt, torch_dev, cache, mirror, rng, start, H, KVH, D)
    q_bits, q_f, g_bits, g_f, k, v = _rand_qkv(rng, M, H, KVH, D)
    got = _prefill(rt, torch_dev, cache, q_bits, g_bits, k, v, H)
    mirror.append(k, v)
    assert cache.sequence_length == start + M
    assert_bf16_close(got, mirror.reference(q_f, g_f, start), what=f"prefill start {start} M {M}")
    _check_cache(cache, mirror)


def test_prefill_equals_decode_steps(rt, torch_dev):
    D, H, KVH, M = 256, 24, 4, 37
    rng = np.random.default_rng(5)
    q_bits, q_f, g_bits, g_f, k, v = _rand_qkv(rng, M, H, KVH, D)
    a = rt.create_q8_kv_state(KVH, D, 64)
    b = rt.create_q8_kv_state(KVH, D, 64)
    pre = _prefill(rt, torch_dev, a, q_bits, g_bits, k, v, H)
    steps = np.concatenate([_decode(rt, torch_dev, [b], q_bits[t:t + 1], g_bits[t:t + 1], k[t], v[t], H)
                            for t in range(M)])
    ka, va, ksa, vsa = a.read()
    kb, vb, ksb, vsb = b.read()
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    assert np.array_equal(ksa, ksb) and np.array_equal(vsa, vsb)
    scale = np.max(np.abs(steps))
    assert np.max(np.abs(pre - steps)) <= scale * (2e-3 + 2 ** -7)


def test_page_table_matches_logical_page_table(rt, torch_dev):
    D, H, KVH = 64, 4, 2
    rng = np.random.default_rng(9)
    cache = rt.create_q8_kv_state(KVH, D, 200)
    ref = oracle.LogicalPageTable(200, 16)
    mirror = Mirror(KVH, D)
    for kind, n in [("prefill", 5), ("decode", 1), ("reserve", 30), ("prefill", 20), ("truncate", 18),
                    ("decode", 1), ("prefill", 40), ("reserve", 0), ("decode", 1)]:
        if kind == "prefill":
            _fill(rt, torch_dev, cache, mirror, rng, n, H, KVH, D)
            ref.append(n)
        elif kind == "decode":
            q_bits, q_f, _, _, k, v = _rand_qkv(rng, 1, H, KVH, D, gate=False)
            got = _decode(rt, torch_dev, [cache], q_bits, None, k, v, H)
            mirror.append(k, v)
            ref.append(1)
            assert_bf16_close(got, mirror.reference(q_f, None, mirror.k.shape[0] - 1), what="after " + kind)
        elif kind == "reserve":
            cache.reserve(n)
            # reserve materialises the pages of [len, len+n) without moving the end
            if n:
                ref.append(n)
                ref.sequence_tokens -= n
        else:
            cache.truncate(n)
            mirror.truncate(n)
            ref.sequence_tokens = n
        assert cache.sequence_length == ref.sequence_tokens
        assert cache.allocated_pages == ref.allocated_pages()
        for t in range(ref.sequence_tokens + 2):
            assert cache.page_for_token(t) == ref.page_for_token(t), (kind, t)
    _check_cache(cache, mirror)


def test_clone_and_truncate(rt, torch_dev):
    D, H, KVH = 128, 8, 2
    rng = np.random.default_rng(11)
    a = rt.create_q8_kv_state(KVH, D, 128)
    ma = Mirror(KVH, D)
    _fill(rt, torch_dev, a, ma, rng, 45, H, KVH, D)
    b = a.clone()
    assert b.sequence_length == 45 and b.allocated_pages == a.allocated_pages
    _check_cache(b, ma)
    b.truncate(30)
    mb = Mirror(KVH, D)
    mb.append(ma.k[:30], ma.v[:30])
    with pytest.raises(QmError, match="INVALID_SEQUENCE_LENGTH"):
        b.truncate(31)
    for m, c in ((ma, a), (mb, b)):
        q_bits, q_f, g_bits, g_f, k, v = _rand_qkv(rng, 3, H, KVH, D)
        got = _prefill(rt, torch_dev, c, q_bits, g_bits, k, v, H)
        start = m.k.shape[0]
        m.append(k, v)
        assert_bf16_close(got, m.reference(q_f, g_f, start), what="after clone/truncate")
        _check_cache(c, m)


@pytest.mark.parametrize("T", [4096, 32768])
def test_long_context_decode(rt, torch_dev, T):
    D, H, KVH = 256, 24, 4
    rng = np.random.default_rng(T)
    cache = rt.create_q8_kv_state(KVH, D, T)
    mirror = Mirror(KVH, D)
    for n in (T - 1) // 4096 * [4096] + [(T - 1) % 4096]:
        _fill(rt, torch_dev, cache, mirror, rng, n, H, KVH, D)
    q_bits, q_f, g_bits, g_f, k, v = _rand_qkv(rng, 1, H, KVH, D)
    got = _decode(rt, torch_dev, [cache], q_bits, g_bits, k, v, H)
    mirror.append(k, v)
    assert_bf16_close(got, mirror.reference(q_f, g_f, T - 1), what=f"T={T}")


def test_rejects_bad_shapes(rt, torch_dev):
    with pytest.raises(QmError, match="INVALID_ATTENTION_SHAPE"):
        rt.create_q8_kv_state(2, 96, 16)
    with pytest.raises(QmError, match="INVALID_ATTENTION_SHAPE"):
        rt.create_q8_kv_state(0, 128, 16)
    with pytest.raises(QmError, match="ZERO_CAPACITY"):
        rt.create_q8_kv_state(2, 128, 0)
    cache = rt.create_q8_kv_state(4, 64, 16)
    q_bits, _, _, _, k, v = _rand_qkv(np.random.default_rng(1), 1, 6, 4, 64, gate=False)
    with pytest.raises(QmError, match="INVALID_ATTENTION_SHAPE"):
        _decode(rt, torch_dev, [cache], q_bits, None, k, v, 6)
    assert cache.sequence_length == 0
