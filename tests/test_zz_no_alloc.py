"""The no-allocation decode attention entry point (qm_attn_decode_noalloc)
against qm_attn_decode, through the C ABI.

The two entry points share the decode and combine kernels and the split
plan; only the split partials' home differs (the library's fixed per-GPU
device array instead of the runtime's grown buffer).  Outputs and cache
bytes must therefore be bit-identical.  Two calls in a row, the second with a
smaller batch and shorter sequences, so the array keeps the first call's
contents when the second reads it.  Also: the caches are not grown (a full
cache is refused), and a plan needing more partials than the array holds is
refused, both without touching the caches; and calls from two streams are
ordered by the library instead of racing on the shared array.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from gpu_util import bf16_dev_to_f32, empty_bf16, to_dev, tuned
from qm38 import QmError, synth

pytestmark = pytest.mark.gpu

H, KVH, D = 64, 8, 128


def _inputs(rng, B):
    q = synth.f32_to_bf16(rng.standard_normal((B, H, D)).astype(np.float32))
    g = synth.f32_to_bf16(rng.standard_normal((B, H, D)).astype(np.float32))
    k = rng.standard_normal((B, KVH, D)).astype(np.float32)
    v = rng.standard_normal((B, KVH, D)).astype(np.float32)
    return q, g, k, v


def _fill(rt, dev, cache, rng, n):
    q, _, k, v = _inputs(rng, n)
    o = empty_bf16((n, H, D), dev)
    rt.gqa_attention_q8_prefill(cache, to_dev(q, dev), None, to_dev(k, dev), to_dev(v, dev), H, n, o)


def _pair(rt, dev, rng, lens):
    """Two identical sets of caches (one per entry point) with room for one more token each."""
    a, b = [], []
    for n in lens:
        c = rt.create_q8_kv_state(KVH, D)
        c.reserve(n + 1)
        c.truncate(0)
        _fill(rt, dev, c, rng, n)
        a.append(c)
        b.append(c.clone())
    return a, b


def _decode(fn, dev, caches, q, g, k, v):
    o = empty_bf16((len(caches), H, D), dev)
    fn(caches, to_dev(q, dev), to_dev(g, dev), to_dev(k, dev), to_dev(v, dev), H, o)
    return bf16_dev_to_f32(o)


def test_noalloc_matches_decode_twice(rt, torch_dev):
    rng = np.random.default_rng(707)
    for lens in ([300, 5000, 17, 40000, 1], [260, 33]):  # second call: smaller batch, shorter sequences
        a, b = _pair(rt, torch_dev, rng, lens)
        q, g, k, v = _inputs(rng, len(lens))
        want = _decode(rt.gqa_attention_q8, torch_dev, a, q, g, k, v)
        got = _decode(rt.gqa_attention_q8_noalloc, torch_dev, b, q, g, k, v)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), lens
        for x, y in zip(a, b):
            assert x.sequence_length == y.sequence_length
            for u, w in zip(x.read(), y.read()):
                assert np.array_equal(u, w)
        for c in a + b:
            c.close()


def test_noalloc_calls_on_two_streams_do_not_overlap(rt, torch_dev):
    """Two runtimes on two streams call the entry point back to back with no
    host synchronisation between them.  Both calls share the GPU's array;
    the library makes the second stream wait for the first call, so each
    output equals its allocating twin's bit for bit."""
    import torch
    rng = np.random.default_rng(710)
    a1, b1 = _pair(rt, torch_dev, rng, [30000, 700])
    a2, b2 = _pair(rt, torch_dev, rng, [20000, 9000])
    in1, in2 = _inputs(rng, 2), _inputs(rng, 2)
    want1 = _decode(rt.gqa_attention_q8, torch_dev, a1, *in1)
    want2 = _decode(rt.gqa_attention_q8, torch_dev, a2, *in2)
    d1 = [to_dev(t, torch_dev) for t in in1]
    d2 = [to_dev(t, torch_dev) for t in in2]
    o1, o2 = empty_bf16((2, H, D), torch_dev), empty_bf16((2, H, D), torch_dev)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    with tuned() as r1, tuned() as r2:
        r1.set_stream(s1)
        r2.set_stream(s2)
        r1.gqa_attention_q8_noalloc(b1, *d1, H, o1)
        r2.gqa_attention_q8_noalloc(b2, *d2, H, o2)
        torch.cuda.synchronize()
    assert np.array_equal(bf16_dev_to_f32(o1).view(np.uint32), want1.view(np.uint32))
    assert np.array_equal(bf16_dev_to_f32(o2).view(np.uint32), want2.view(np.uint32))
    for c in a1 + b1 + a2 + b2:
        c.close()


def test_noalloc_refuses_growth_and_oversized_plans(rt, torch_dev):
    rng = np.random.default_rng(708)
    full = rt.create_q8_kv_state(KVH, D)
    _fill(rt, torch_dev, full, rng, 16)  # capacity 16, all used
    q, g, k, v = _inputs(rng, 1)
    with pytest.raises(QmError, match="CAPACITY_EXCEEDED"):
        _decode(rt.gqa_attention_q8_noalloc, torch_dev, [full], q, g, k, v)
    assert full.sequence_length == 16 and full.capacity_tokens == 16
    # Splits of 4 pages over 40000 tokens: 625 splits x 64 heads x 130 floats
    # = 20.8 MB of partials, more than the 16 MiB array.
    big = rt.create_q8_kv_state(KVH, D)
    big.reserve(40001)
    big.truncate(0)
    _fill(rt, torch_dev, big, rng, 40000)
    with tuned(QM38_ATTN_PPS=4) as trt:
        with pytest.raises(QmError, match="CAPACITY_EXCEEDED"):
            _decode(trt.gqa_attention_q8_noalloc, torch_dev, [big], q, g, k, v)
    assert big.sequence_length == 40000
    # The default plan of the same call fits.
    got = _decode(rt.gqa_attention_q8_noalloc, torch_dev, [big], q, g, k, v)
    assert big.sequence_length == 40001 and np.all(np.isfinite(got))


def test_noalloc_allocates_no_device_memory(rt, torch_dev):
    # The entry point's contract: no device allocation, measured as the
    # device's free bytes around a call on a runtime that has never allocated
    # a workspace.  The control (qm_attn_decode on another such runtime,
    # planned with splits of 4 pages so that its partials take 20.8 MB) shows
    # that the measurement sees an allocation of that size.
    import torch
    rng = np.random.default_rng(709)
    a, b = _pair(rt, torch_dev, rng, [40000])
    c, d = _pair(rt, torch_dev, rng, [40000])
    q, g, k, v = _inputs(rng, 1)
    qd, gd, kd, vd = (to_dev(t, torch_dev) for t in (q, g, k, v))
    o = empty_bf16((1, H, D), torch_dev)
    # The library's code object (with its fixed array) is loaded by earlier
    # calls in this process; warm the symbol lookup once more on its own.
    rt.gqa_attention_q8_noalloc(d, qd, gd, kd, vd, H, o)
    torch.cuda.synchronize()

    def free_bytes():
        torch.cuda.synchronize()
        return torch.cuda.mem_get_info()[0]

    with tuned() as fresh:
        before = free_bytes()
        fresh.gqa_attention_q8_noalloc(b, qd, gd, kd, vd, H, o)
        after = free_bytes()
    with tuned(QM38_ATTN_PPS=4) as control:  # 625 splits: 20.8 MB of partials
        c_before = free_bytes()
        control.gqa_attention_q8(c, qd, gd, kd, vd, H, o)
        c_after = free_bytes()
    if c_before - c_after < (16 << 20):
        pytest.skip(f"free-memory reading did not see the control's allocation ({c_before - c_after} B)")
    assert before == after, f"qm_attn_decode_noalloc changed free device memory by {before - after} B"
    for x in a + b + c + d:
        x.close()
