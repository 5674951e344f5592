"""GPU parity of the paged Q8-KV GQA attention against the CPU oracle.

Ports metal_runtime.rs tests q8_gqa_attention_keeps_kv_on_the_gpu (:11587),
q8_gqa_prefill_matches_steps_and_keeps_kv_state (:11608) and
q8_gqa_prefill_matches_steps_when_kv_capacity_grows (:11683) at their own
head_dim 2 and with the reference's capacity growth, plus seeded cases at
the model's shapes (head_dim 256, GQA groups up to 16, ragged batches,
split-K decode), odd head dimensions, and BASELINE config 4 at 64 query /
8 KV heads, d = 128: decode at 128K, a ragged batch of 8 over
{4K, 32K, 128K} and a 2048-row causal prefill onto a 4096-token cache.

Bars: quantised cache bytes and scales bit-exact against the oracle's
quantiser; page tables identical to LogicalPageTable; outputs (bf16) within
1e-4 of max|ref| beyond bf16 rounding, against an fp64-accumulated oracle
fed the same bf16 q and gate.
"""
from __future__ import annotations

import math
import os

import numpy as np
import pytest

import oracle
import torch
from gpu_util import assert_bf16_close, bf16_dev_to_f32, bf16_half_ulp, empty_bf16, to_dev, tuned
from qm38 import QmError, synth

pytestmark = pytest.mark.gpu


class Mirror:
    """Host copy of one sequence's appended fp32 K/V rows."""

    def __init__(self, kvh, d):
        self.kvh, self.d = kvh, d
        self._k, self._v = [np.zeros((0, kvh, d), np.float32)], [np.zeros((0, kvh, d), np.float32)]

    def append(self, k, v):
        self._k.append(np.asarray(k, np.float32).reshape(-1, self.kvh, self.d))
        self._v.append(np.asarray(v, np.float32).reshape(-1, self.kvh, self.d))

    @property
    def k(self):
        if len(self._k) > 1:
            self._k = [np.concatenate(self._k)]
        return self._k[0]

    @property
    def v(self):
        if len(self._v) > 1:
            self._v = [np.concatenate(self._v)]
        return self._v[0]

    def truncate(self, n):
        self._k, self._v = [self.k[:n]], [self.v[:n]]

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
# Reference known-answer tests (head_dim 2, as the reference runs them)
# ---------------------------------------------------------------------------
KAT_D = 2


def _pad(a, heads):
    return np.asarray(a, np.float32).reshape(-1, heads, KAT_D)


def test_reference_kat_single_token(rt, torch_dev):
    # metal_runtime.rs:11587-11605
    cache = rt.create_q8_kv_state(1, KAT_D, 64)
    q_bits, _ = _bf16(_pad([1.0, 0.0], 1))
    g_bits, _ = _bf16(_pad([0.0, 0.0], 1))
    out = _decode(rt, torch_dev, [cache], q_bits, g_bits, _pad([1.0, 0.0], 1), _pad([2.0, -1.0], 1), 1)
    assert cache.sequence_length == 1
    assert abs(out[0, 0, 0] - 1.0) < 0.001, out[0, 0, :2]
    assert abs(out[0, 0, 1] + 0.5) < 0.005, out[0, 0, :2]
    keys, values, ks, vs = cache.read()
    assert list(values[0, 0, :2]) == [127, -64] and ks[0, 0] == np.float32(1.0) / np.float32(127.0)
    assert vs[0, 0] == np.float32(2.0) / np.float32(127.0)


def test_reference_kat_prefill_matches_steps(rt, torch_dev):
    # metal_runtime.rs:11608-11682 (H=2, KVH=1)
    queries = [1.0, 0.0, 0.25, -0.5, 0.5, 0.5, -0.75, 0.25, -0.2, 0.8, 0.6, -0.4]
    gates = [0.0, 0.0, 0.1, -0.1, -0.2, 0.2, 0.0, 0.0, 0.3, -0.3, 0.15, 0.05]
    keys = [1.0, 0.0, 0.4, 0.9, -0.7, 0.2]
    values = [2.0, -1.0, 0.75, 1.25, -0.5, 0.4]
    q_bits, q_f = _bf16(_pad(queries, 2))
    g_bits, g_f = _bf16(_pad(gates, 2))
    k, v = _pad(keys, 1), _pad(values, 1)
    step = rt.create_q8_kv_state(1, KAT_D, 64)
    pre = rt.create_q8_kv_state(1, KAT_D, 64)
    expected = np.concatenate([_decode(rt, torch_dev, [step], q_bits[t:t + 1], g_bits[t:t + 1], k[t], v[t], 2)
                               for t in range(3)])
    actual = _prefill(rt, torch_dev, pre, q_bits, g_bits, k, v, 2)
    assert pre.sequence_length == 3
    assert np.max(np.abs(actual - expected)) < 0.005
    mirror = Mirror(1, KAT_D)
    mirror.append(k, v)
    assert_bf16_close(actual, mirror.reference(q_f, g_f, 0), what="kat prefill")
    _check_cache(pre, mirror)
    _check_cache(step, mirror)

    nq_bits, nq_f = _bf16(_pad([0.9, -0.1, -0.3, 0.7], 2))
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
    q_bits, q_f = _bf16(_pad([x for r in rows for x in r[0]], 2))
    g_bits, g_f = _bf16(_pad([x for r in rows for x in r[1]], 2))
    k = _pad([x for r in rows for x in r[2]], 1)
    v = _pad([x for r in rows for x in r[3]], 1)
    step = rt.create_q8_kv_state(1, KAT_D)
    pre = rt.create_q8_kv_state(1, KAT_D)
    assert step.capacity_tokens == pre.capacity_tokens == 16
    for t in range(16):
        _decode(rt, torch_dev, [step], q_bits[t:t + 1], g_bits[t:t + 1], k[t], v[t], 2)
    _prefill(rt, torch_dev, pre, q_bits[:16], g_bits[:16], k[:16], v[:16], 2)
    mirror = Mirror(1, KAT_D)
    mirror.append(k[:16], v[:16])
    _check_cache(step, mirror)
    _check_cache(pre, mirror)
    assert step.capacity_tokens == pre.capacity_tokens == 16
    step.reserve(3)
    pre.reserve(3)
    # ensure_q8_kv_capacity: next power of two of 19 tokens, pages copied
    assert step.capacity_tokens == pre.capacity_tokens == 32
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


def test_capacity_grows_on_append_and_respects_hard_limit(rt, torch_dev):
    """Appends past the capacity grow the cache without a reserve (decode and
    prefill); a cache created with a hard token limit (LogicalPageTable's
    capacity) refuses to pass it and leaves its state unchanged."""
    D, H, KVH = 128, 8, 2
    rng = np.random.default_rng(21)
    cache = rt.create_q8_kv_state(KVH, D)
    mirror = Mirror(KVH, D)
    for n in (15, 1, 1, 40):  # 16 -> 32 (decode) -> 64 (prefill of 40)
        if n == 1:
            q_bits, q_f, g_bits, g_f, k, v = _rand_qkv(rng, 1, H, KVH, D)
            got = _decode(rt, torch_dev, [cache], q_bits, g_bits, k, v, H)
        else:
            q_bits, q_f, g_bits, g_f, k, v = _rand_qkv(rng, n, H, KVH, D)
            got = _prefill(rt, torch_dev, cache, q_bits, g_bits, k, v, H)
        start = mirror.k.shape[0]
        mirror.append(k, v)
        assert_bf16_close(got, mirror.reference(q_f, g_f, start), what=f"after growth to {cache.capacity_tokens}")
    assert cache.capacity_tokens == 64 and cache.sequence_length == 57
    _check_cache(cache, mirror)
    lim = rt.create_q8_kv_state(KVH, D, 20)
    q_bits, q_f, g_bits, g_f, k, v = _rand_qkv(rng, 20, H, KVH, D)
    _prefill(rt, torch_dev, lim, q_bits, g_bits, k, v, H)
    assert lim.capacity_tokens == 20
    with pytest.raises(QmError, match="CAPACITY_EXCEEDED"):
        _decode(rt, torch_dev, [lim], q_bits[:1], g_bits[:1], k[0], v[0], H)
    with pytest.raises(QmError, match="CAPACITY_EXCEEDED"):
        lim.reserve(1)
    assert lim.sequence_length == 20 and lim.allocated_pages == 2


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
@pytest.mark.parametrize("waves", [4, 8])
def test_decode_ragged_batch(rt, torch_dev, D, H, KVH, pps, waves):
    # Both workgroup shapes of the decode kernel (two 4-wave workgroups per
    # CU, or one 8-wave workgroup), whichever the planner would pick.
    rng = np.random.default_rng(D * 7 + H * 3 + KVH + pps)
    lens = [0, 15, 16, 17, 100, 333]
    caches = [rt.create_q8_kv_state(KVH, D, 512) for _ in lens]
    mirrors = [Mirror(KVH, D) for _ in lens]
    for c, m, n in zip(caches, mirrors, lens):
        _fill(rt, torch_dev, c, m, rng, n, H, KVH, D)
    with tuned(QM38_ATTN_PPS=pps or None, QM38_ATTN_WAVES=waves) as trt:
        for it in range(2):
            q_bits, q_f, g_bits, g_f, k, v = _rand_qkv(rng, len(lens), H, KVH, D, gate=(it == 0))
            got = _decode(trt, torch_dev, caches, q_bits, g_bits, k, v, H)
            for b, (c, m) in enumerate(zip(caches, mirrors)):
                m.append(k[b], v[b])
                assert c.sequence_length == m.k.shape[0]
                ref = m.reference(q_f[b:b + 1], None if g_f is None else g_f[b:b + 1], m.k.shape[0] - 1)
                assert_bf16_close(got[b:b + 1], ref, what=f"seq {b} len {m.k.shape[0]} it {it}")
    for c, m in zip(caches, mirrors):
        _check_cache(c, m)


@pytest.mark.parametrize("D,H,KVH", [(128, 64, 8), (64, 8, 8)])
@pytest.mark.parametrize("waves,pps", [(4, 320), (8, 576)])
def test_decode_long_split_page_ids(rt, torch_dev, D, H, KVH, waves, pps):
    """Waves past 64 pages of their split: the first 64 ids come from the
    per-wave id vector, the rest from scalar loads.  4 waves, splits of 320
    pages: 80 pages a wave, and the page this step materialises, page 620, is
    wave 0's 76th page of split 1.  8 waves, splits of 576 pages: 72 pages a
    wave in split 0."""
    rng = np.random.default_rng(D + H)
    n = 620 * 16
    cache = rt.create_q8_kv_state(KVH, D, n + 64)
    mirror = Mirror(KVH, D)
    _fill(rt, torch_dev, cache, mirror, rng, n, H, KVH, D)
    with tuned(QM38_ATTN_PPS=pps, QM38_ATTN_WAVES=waves) as trt:
        for it in range(2):
            q_bits, q_f, g_bits, g_f, k, v = _rand_qkv(rng, 1, H, KVH, D, gate=(it == 1))
            got = _decode(trt, torch_dev, [cache], q_bits, g_bits, k, v, H)
            mirror.append(k[0], v[0])
            ref = mirror.reference(q_f, g_f, mirror.k.shape[0] - 1)
            assert_bf16_close(got, ref, what=f"len {mirror.k.shape[0]} it {it}")
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
    # Two bf16 results of the same math: apart by at most their two output
    # roundings plus 1e-4 of max|out|.
    scale = np.max(np.abs(steps))
    slack = bf16_half_ulp(pre) + bf16_half_ulp(steps)
    assert np.max(np.abs(pre - steps) - slack) <= 1e-4 * scale


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


@pytest.mark.parametrize("max_tokens", [20, 5])
def test_clone_at_a_limit_below_the_page_size(rt, torch_dev, max_tokens):
    # A limit that is not a multiple of 16: the pages hold more tokens than
    # the limit allows, and the clone must take the capacity the source may
    # use (clone_q8_kv_state, metal_runtime.rs:7338-7379), also for an empty
    # cache and one filled to the limit.
    D, H, KVH = 64, 4, 2
    rng = np.random.default_rng(max_tokens)
    a = rt.create_q8_kv_state(KVH, D, max_tokens)
    e = a.clone()
    assert e.sequence_length == 0
    ma = Mirror(KVH, D)
    _fill(rt, torch_dev, a, ma, rng, max_tokens, H, KVH, D)
    assert a.sequence_length == max_tokens and a.capacity_tokens == max_tokens
    b = a.clone()
    assert b.sequence_length == max_tokens and b.capacity_tokens == max_tokens
    _check_cache(b, ma)
    with pytest.raises(QmError, match="CAPACITY_EXCEEDED"):
        b.reserve(1)
    b.truncate(max_tokens - 2)
    mb = Mirror(KVH, D)
    mb.append(ma.k[:max_tokens - 2], ma.v[:max_tokens - 2])
    q_bits, q_f, g_bits, g_f, k, v = _rand_qkv(rng, 2, H, KVH, D)
    got = _prefill(rt, torch_dev, b, q_bits, g_bits, k, v, H)
    mb.append(k, v)
    assert_bf16_close(got, mb.reference(q_f, g_f, max_tokens - 2), what="clone at the limit")
    _check_cache(b, mb)


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
    # validate_attention_shape (metal_runtime.rs:9186-9193): 1 <= head_dim <= 256, kv_heads > 0
    with pytest.raises(QmError, match="INVALID_ATTENTION_SHAPE"):
        rt.create_q8_kv_state(2, 257)
    with pytest.raises(QmError, match="INVALID_ATTENTION_SHAPE"):
        rt.create_q8_kv_state(2, 0)
    with pytest.raises(QmError, match="INVALID_ATTENTION_SHAPE"):
        rt.create_q8_kv_state(0, 128, 16)
    cache = rt.create_q8_kv_state(4, 64, 16)
    q_bits, _, _, _, k, v = _rand_qkv(np.random.default_rng(1), 1, 6, 4, 64, gate=False)
    with pytest.raises(QmError, match="INVALID_ATTENTION_SHAPE"):
        _decode(rt, torch_dev, [cache], q_bits, None, k, v, 6)
    assert cache.sequence_length == 0


# ---------------------------------------------------------------------------
# Head dimensions other than the kernel widths (pages padded with zeros)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("D,H,KVH", [(1, 2, 1), (2, 4, 2), (33, 6, 3), (80, 16, 2), (96, 8, 4), (200, 8, 1),
                                      (255, 4, 4)])
def test_odd_head_dims(rt, torch_dev, D, H, KVH):
    rng = np.random.default_rng(D * 31 + H)
    lens = [0, 17, 300]
    caches = [rt.create_q8_kv_state(KVH, D) for _ in lens]
    mirrors = [Mirror(KVH, D) for _ in lens]
    for c, m, n in zip(caches, mirrors, lens):
        if n:
            q_bits, q_f, g_bits, g_f, k, v = _rand_qkv(rng, n, H, KVH, D)
            got = _prefill(rt, torch_dev, c, q_bits, g_bits, k, v, H)
            m.append(k, v)
            assert_bf16_close(got, m.reference(q_f, g_f, 0), what=f"prefill d={D} n={n}")
    with tuned(QM38_ATTN_PPS=4) as trt:  # split the 300-token cache: the merge runs
        q_bits, q_f, g_bits, g_f, k, v = _rand_qkv(rng, len(lens), H, KVH, D)
        got = _decode(trt, torch_dev, caches, q_bits, g_bits, k, v, H)
    for b, (c, m) in enumerate(zip(caches, mirrors)):
        m.append(k[b], v[b])
        ref = m.reference(q_f[b:b + 1], g_f[b:b + 1], m.k.shape[0] - 1)
        assert_bf16_close(got[b:b + 1], ref, what=f"decode d={D} seq {b}")
        _check_cache(c, m)


# ---------------------------------------------------------------------------
# 64 query heads, 8 KV heads, head_dim 128
# ---------------------------------------------------------------------------
C4_H, C4_KVH, C4_D = 64, 8, 128


def _fill_device(rt, dev, cache, mirror, gen, n, KVH, D, chunk=8192):
    """Appends n N(0,1) K/V rows drawn on the GPU (prefill with one query head
    per KV head, outputs unused), mirrored on the host."""
    done = 0
    while done < n:
        m = min(chunk, n - done)
        k = torch.randn((m, KVH, D), generator=gen, device=dev, dtype=torch.float32)
        v = torch.randn((m, KVH, D), generator=gen, device=dev, dtype=torch.float32)
        q = torch.zeros((m, KVH, D), dtype=torch.int16, device=dev)
        o = torch.empty((m, KVH, D), dtype=torch.int16, device=dev)
        rt.gqa_attention_q8_prefill(cache, q, None, k, v, KVH, m, o)
        mirror.append(k.cpu().numpy(), v.cpu().numpy())
        done += m


def test_config4_decode_128k(rt, torch_dev):
    gen = torch.Generator(device=torch_dev)
    gen.manual_seed(4128)
    rng = np.random.default_rng(4128)
    T = 131072
    cache = rt.create_q8_kv_state(C4_KVH, C4_D)
    mirror = Mirror(C4_KVH, C4_D)
    _fill_device(rt, torch_dev, cache, mirror, gen, T - 1, C4_KVH, C4_D)
    for it in range(2):
        q_bits, q_f, g_bits, g_f, k, v = _rand_qkv(rng, 1, C4_H, C4_KVH, C4_D)
        got = _decode(rt, torch_dev, [cache], q_bits, g_bits, k, v, C4_H)
        mirror.append(k, v)
        assert_bf16_close(got, mirror.reference(q_f, g_f, mirror.k.shape[0] - 1), what=f"128K decode it {it}")
    assert cache.sequence_length == T + 1


def test_config4_ragged_batch(rt, torch_dev):
    """B = 8 sequences whose lengths are drawn (seeded) from {4K, 32K, 128K}."""
    gen = torch.Generator(device=torch_dev)
    gen.manual_seed(48)
    rng = np.random.default_rng(48)
    lens = [int(x) for x in rng.choice([4096, 32768, 131072], size=8)]
    lens[0], lens[1], lens[2] = 4096, 32768, 131072  # every length present
    caches = [rt.create_q8_kv_state(C4_KVH, C4_D) for _ in lens]
    mirrors = [Mirror(C4_KVH, C4_D) for _ in lens]
    for c, m, n in zip(caches, mirrors, lens):
        _fill_device(rt, torch_dev, c, m, gen, n - 1, C4_KVH, C4_D)
    q_bits, q_f, g_bits, g_f, k, v = _rand_qkv(rng, len(lens), C4_H, C4_KVH, C4_D)
    got = _decode(rt, torch_dev, caches, q_bits, g_bits, k, v, C4_H)
    for b, (c, m) in enumerate(zip(caches, mirrors)):
        m.append(k[b], v[b])
        assert c.sequence_length == lens[b]
        ref = m.reference(q_f[b:b + 1], g_f[b:b + 1], lens[b] - 1)
        assert_bf16_close(got[b:b + 1], ref, what=f"ragged seq {b} len {lens[b]}")
        keys, values, ks, vs = c.read()
        kq, kss, vq, vss = m.quantised()
        assert np.array_equal(keys[-1], kq[-1]) and np.array_equal(values[-1], vq[-1])
        assert np.array_equal(ks[-1], kss[-1]) and np.array_equal(vs[-1], vss[-1])
        mirrors[b] = None  # free host memory early


def test_config4_prefill_2048_on_4k(rt, torch_dev):
    """2048 new rows appended to a 4096-token cache; every cache byte checked,
    outputs of 40 rows (the first, last and a seeded sample) against the oracle."""
    gen = torch.Generator(device=torch_dev)
    gen.manual_seed(2048)
    rng = np.random.default_rng(2048)
    cache = rt.create_q8_kv_state(C4_KVH, C4_D)
    mirror = Mirror(C4_KVH, C4_D)
    _fill_device(rt, torch_dev, cache, mirror, gen, 4096, C4_KVH, C4_D)
    M = 2048
    q_bits, q_f, g_bits, g_f, k, v = _rand_qkv(rng, M, C4_H, C4_KVH, C4_D)
    got = _prefill(rt, torch_dev, cache, q_bits, g_bits, k, v, C4_H)
    mirror.append(k, v)
    assert cache.sequence_length == 4096 + M
    _check_cache(cache, mirror)
    kq, ks, vq, vs = mirror.quantised()
    rows = sorted(set([0, 1, 15, 16, M - 1] + [int(r) for r in rng.choice(M, size=35, replace=False)]))
    for r in rows:
        ref = oracle.attention(q_f[r:r + 1], g_f[r:r + 1], kq, ks, vq, vs, 4096 + r)
        assert_bf16_close(got[r:r + 1], ref, what=f"prefill row {r}")
