"""qm38 benchmark: the reference's per-token compute path on one MI355X.

Headline (`value`): MLX affine-Q4 decode projection set at 27B-class shapes
with one activation row: fused QKV 5120->10240, gate+up
5120->2x17408 with SwiGLU in the epilogue, down 17408->5120.  One step = one
pass of the three projections; `value` = algorithmic bytes of the step / step
time (GB/s), inputs resident in HBM.  Three copies of the weights (540 MB)
rotate between steps so the 256 MB MALL cannot serve them.

`extras` carries the other legs of the metric, each against its roofline:
the decode set at 4 and 8 rows; Q8-KV decode attention at 32K context
(us/token) and a ragged batch of 8 sequences over {4K, 32K, 128K}; causal
prefill attention (2048 rows onto a 4K cache); the Q4 prefill GEMM set at
M = 512 and 2048 (TFLOP/s); the Gated DeltaNet decode step and 2048-token
prefill.  `roofline` describes the dominant kernel of the headline (the
gate+up SwiGLU projection), timed with HIP events on the stream it is
launched on.  `cpu_baseline` runs the same decode-projection math on host
cores (oracle/, OpenMP) over a bounded sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu]
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "qwen38-metal_amd"))

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, GB/s
MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 / bf16 MFMA, TFLOP/s
FP32_PEAK_TFLOPS = 157.3   # MI355X dense fp32 (matrix), TFLOP/s

H, I, QKV = 5120, 17408, 10240
ATT_H, ATT_KVH, ATT_D = 64, 8, 128
DN = dict(key_heads=16, value_heads=32, key_head_dim=128, value_head_dim=128, conv_kernel_size=4)
NCOPY = 3


def q4_bytes(rows: int, cols: int) -> int:
    return rows * cols // 2 + 2 * rows * (cols // 64) * 2


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def dev_array(a, dev):
    import torch
    a = np.ascontiguousarray(a)
    v = {np.dtype(np.uint16): np.int16, np.dtype(np.uint32): np.int32}.get(a.dtype)
    return torch.from_numpy(a.view(v) if v is not None else a).to(dev)


class Events:
    """HIP events recorded on the stream the kernels are launched on."""

    def __init__(self, stream):
        import torch
        self.torch = torch
        self.stream = stream

    def mark(self):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record(self.stream)
        return e


_BLOCK = {}


def gpu_blocker(ms: float = 12.0):
    """Queues ~ms of unrelated GPU work so that the host enqueues the timed
    steps while the GPU is busy: the events then see the kernels back to back
    instead of waiting on Python launch overhead."""
    import torch
    if "a" not in _BLOCK:
        _BLOCK["a"] = torch.randn((4096, 4096), dtype=torch.float16, device="cuda")
        a = _BLOCK["a"]
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(4):
            torch.mm(a, a)
        e1.record()
        torch.cuda.synchronize()
        _BLOCK["n"] = max(1, int(ms / max(e0.elapsed_time(e1) / 4, 1e-3)))
    a = _BLOCK["a"]
    for _ in range(_BLOCK["n"]):
        torch.mm(a, a)


def timed(step, stream, steps: int, warmup: int):
    """Runs warmup + steps calls of step(i, marks); returns (ms per step, per-step mark lists)."""
    import torch
    ev = Events(stream)
    for i in range(warmup):
        step(i, None)
    torch.cuda.synchronize()
    gpu_blocker()
    marks_all = []
    t0 = ev.mark()
    for i in range(steps):
        marks = [ev]
        step(warmup + i, marks)
        marks_all.append(marks[1:])
    t1 = ev.mark()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps, marks_all


def step_distribution(step, stream, steps: int, warmup: int = 2):
    """Per-step times (us) from one event after each step: (p10, median, p90).
    The events sit between steps, so the set's own kernels stay back to back."""
    import torch
    ev = Events(stream)
    for i in range(warmup):
        step(i, None)
    torch.cuda.synchronize()
    gpu_blocker()
    marks = [ev.mark()]
    for i in range(steps):
        step(warmup + i, None)
        marks.append(ev.mark())
    torch.cuda.synchronize()
    d = np.array([a.elapsed_time(b) * 1e3 for a, b in zip(marks[:-1], marks[1:])])
    return tuple(round(float(v), 2) for v in np.percentile(d, [10, 50, 90]))


# ---------------------------------------------------------------------------
# Q4 projections
# ---------------------------------------------------------------------------
def synth_bf16(rng, shape):
    from qm38 import synth
    return synth.bf16_normal(rng, shape)


def q4_sets(rng, dev):
    import qm38
    from qm38 import synth
    sets = []
    for _ in range(NCOPY):
        mats = {}
        for name, rows, cols in (("qkv", QKV, H), ("gate", I, H), ("up", I, H), ("down", H, I)):
            w, s, b = synth.q4_matrix(rng, rows, cols)
            t = (dev_array(w, dev), dev_array(s, dev), dev_array(b, dev))
            mats[name] = (qm38.Runtime.job(*t, rows), t)
        sets.append(mats)
    return sets


def q4_leg(rt, dev, sets, M: int, rng, steps, warmup):
    """QKV with gate+up (SwiGLU) as one same-input set, then down, over M rows;
    returns timings and byte / flop counts."""
    import torch
    from qm38 import synth
    x = dev_array(synth.bf16_normal(rng, (M, H)), dev)
    qkv_out = torch.empty((M, QKV), dtype=torch.int16, device=dev)
    h = torch.empty((M, I), dtype=torch.int16, device=dev)
    y = torch.empty((M, H), dtype=torch.int16, device=dev)

    def qkv_gateup(j):
        rt.q4_project_set([j["qkv"][0], j["gate"][0]], [None, j["up"][0]], x, H, M, [qkv_out, h])

    def step(i, marks):
        j = sets[i % NCOPY]
        qkv_gateup(j)
        rt.q4_project([j["down"][0]], h, I, M, [y])

    stream = torch.cuda.current_stream()
    ms, _ = timed(step, stream, steps, warmup)
    # Per-kernel durations: each projection alone, back to back (events only
    # around the whole run, so no event sits between the timed kernels).
    calls = {
        "qkv_gateup": lambda i, m: qkv_gateup(sets[i % NCOPY]),
        "down": lambda i, m: rt.q4_project([sets[i % NCOPY]["down"][0]], h, I, M, [y]),
    }
    per = [timed(fn, stream, steps, 2)[0] for fn in calls.values()]
    wbytes = {"qkv_gateup": q4_bytes(QKV, H) + 2 * q4_bytes(I, H), "down": q4_bytes(H, I)}
    abytes = {"qkv_gateup": 2 * M * (H + QKV + I), "down": 2 * M * (I + H)}
    flops = {"qkv_gateup": 2 * M * QKV * H + 4 * M * I * H, "down": 2 * M * H * I}
    kern = dict(zip(calls, per))
    q4_leg.last_step = step
    return ms, kern, wbytes, abytes, flops


def matvec_4096_leg(rt, dev, rng, steps, warmup):
    """one 4096 x 4096 Q4 matvec (M = 1), launch-bound."""
    import torch
    import qm38
    from qm38 import synth
    N = K = 4096
    jobs = []
    for _ in range(NCOPY):
        w, sc, b = synth.q4_matrix(rng, N, K)
        jobs.append((qm38.Runtime.job(dev_array(w, dev), dev_array(sc, dev), dev_array(b, dev), N)))
    x = dev_array(synth_bf16(rng, (1, K)), dev)
    y = torch.empty((1, N), dtype=torch.int16, device=dev)
    ms, _ = timed(lambda i, m: rt.q4_project([jobs[i % NCOPY]], x, K, 1, [y]), torch.cuda.current_stream(), steps,
                  warmup)
    nbytes = q4_bytes(N, K) + 2 * K + 2 * N  # 9,453,568 B
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"us": round(ms * 1e3, 2), "bytes": nbytes, "GB/s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}


# ---------------------------------------------------------------------------
# Q8-KV attention
# ---------------------------------------------------------------------------
def kv_fill(rt, dev, cache, rng, tokens: int, chunk: int = 8192):
    """Appends `tokens` random K/V rows through the prefill entry point with one
    query head per KV head (the cheapest causal pass; its output is unused)."""
    import torch
    from qm38 import synth
    done = 0
    q = dev_array(synth.bf16_normal(rng, (chunk, ATT_KVH, ATT_D)), dev)
    o = torch.empty((chunk, ATT_KVH, ATT_D), dtype=torch.int16, device=dev)
    kv = torch.randn((2, chunk, ATT_KVH, ATT_D), dtype=torch.float32, device=dev)
    while done < tokens:
        n = min(chunk, tokens - done)
        rt.gqa_attention_q8_prefill(cache, q, None, kv[0], kv[1], ATT_KVH, n, o)
        done += n
    torch.cuda.synchronize()


def kv_cache(rt, tokens: int):
    """A cache grown to hold `tokens` tokens up front (no growth in timed calls)."""
    c = rt.create_q8_kv_state(ATT_KVH, ATT_D)
    c.reserve(tokens)
    c.truncate(0)
    return c


def attn_bytes(T: int) -> int:
    return T * ATT_KVH * ATT_D * 2 + T * ATT_KVH * 2 * 4


def attention_legs(rt, dev, rng, steps, warmup):
    import torch
    from qm38 import synth
    out = {}
    stream = torch.cuda.current_stream()
    # (a) one sequence at 32K: us per decode token.  Six caches (415 MB) take
    # turns so the 256 MB MALL cannot hold the one being read.
    T0, NC = 32768, 6
    caches = []
    for _ in range(NC):
        c = kv_cache(rt, T0 + steps + warmup + 8)
        kv_fill(rt, dev, c, rng, T0)
        caches.append(c)
    q = dev_array(synth.bf16_normal(rng, (1, ATT_H, ATT_D)), dev)
    g = dev_array(synth.bf16_normal(rng, (1, ATT_H, ATT_D)), dev)
    k = torch.randn((1, ATT_KVH, ATT_D), dtype=torch.float32, device=dev)
    v = torch.randn((1, ATT_KVH, ATT_D), dtype=torch.float32, device=dev)
    o = torch.empty((1, ATT_H, ATT_D), dtype=torch.int16, device=dev)
    ms, _ = timed(lambda i, m: rt.gqa_attention_q8([caches[i % NC]], q, g, k, v, ATT_H, o), stream, steps, warmup)
    T_avg = T0 + (warmup + steps) / NC / 2
    gbs = attn_bytes(int(T_avg)) / (ms * 1e-3) / 1e9
    out["attn_decode_32k"] = {"us_per_token": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                              "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                              "shape": f"H=64 KVH=8 d=128, 1 sequence at 32K, {NC} caches in turn"}
    for c in caches:
        c.close()
    torch.cuda.empty_cache()
    # (b) ragged batch of 8 over {4K, 32K, 128K}.
    lens = list(np.random.default_rng(4).choice([4096, 32768, 131072], 8))
    caches = []
    for n in lens:
        c = kv_cache(rt, int(n) + steps + warmup + 8)
        kv_fill(rt, dev, c, rng, int(n))
        caches.append(c)
    B = len(caches)
    q = dev_array(synth.bf16_normal(rng, (B, ATT_H, ATT_D)), dev)
    g = dev_array(synth.bf16_normal(rng, (B, ATT_H, ATT_D)), dev)
    k = torch.randn((B, ATT_KVH, ATT_D), dtype=torch.float32, device=dev)
    v = torch.randn((B, ATT_KVH, ATT_D), dtype=torch.float32, device=dev)
    o = torch.empty((B, ATT_H, ATT_D), dtype=torch.int16, device=dev)
    ms, _ = timed(lambda i, m: rt.gqa_attention_q8(caches, q, g, k, v, ATT_H, o), stream, steps, warmup)
    total = sum(attn_bytes(int(n) + warmup + steps // 2) for n in lens)
    gbs = total / (ms * 1e-3) / 1e9
    out["attn_decode_ragged_b8"] = {"us_per_step": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                                    "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                                    "lengths": [int(n) for n in lens]}
    for c in caches:
        c.close()
    torch.cuda.empty_cache()
    # (c) causal prefill: 2048 rows onto a 4096-token cache.
    P, T = 2048, 4096
    reps = max(2, min(steps, 5))
    caches = [kv_cache(rt, T + P) for _ in range(reps + 1)]
    for c in caches:
        kv_fill(rt, dev, c, rng, T)
    q = dev_array(synth.bf16_normal(rng, (P, ATT_H, ATT_D)), dev)
    g = dev_array(synth.bf16_normal(rng, (P, ATT_H, ATT_D)), dev)
    k = torch.randn((P, ATT_KVH, ATT_D), dtype=torch.float32, device=dev)
    v = torch.randn((P, ATT_KVH, ATT_D), dtype=torch.float32, device=dev)
    o = torch.empty((P, ATT_H, ATT_D), dtype=torch.int16, device=dev)
    ms, _ = timed(lambda i, m: rt.gqa_attention_q8_prefill(caches[i], q, g, k, v, ATT_H, P, o), stream, reps, 1)
    flops = 4.0 * ATT_H * ATT_D * sum(T + i + 1 for i in range(P))
    out["attn_prefill_2048_on_4k"] = {"ms": round(ms, 3), "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 2),
                                      "mfma_frac": round(flops / (ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4)}
    for c in caches:
        c.close()
    torch.cuda.empty_cache()
    # (d) q/k preparation (RMSNorm + RoPE + query/gate split) for 1 and 2048
    # rows, rotary_dim = head_dim / 4 (partial_rotary_factor 0.25).
    import qm38
    rope = qm38.RopeConfig(ATT_D, ATT_D // 4, 1e7, 0, 0, 0)
    qn = torch.ones(ATT_D, dtype=torch.float32, device=dev)
    for R in (1, 2048):
        qg = dev_array(synth.bf16_normal(rng, (R, ATT_H, 2 * ATT_D)), dev)
        kin = dev_array(synth.bf16_normal(rng, (R, ATT_KVH, ATT_D)), dev)
        qo = torch.empty((R, ATT_H, ATT_D), dtype=torch.int16, device=dev)
        go = torch.empty((R, ATT_H, ATT_D), dtype=torch.int16, device=dev)
        ko = torch.empty((R, ATT_KVH, ATT_D), dtype=torch.float32, device=dev)
        ms, _ = timed(lambda i, m: rt.attn_prepare(rope, R, ATT_H, ATT_KVH, qg, kin, qn, qn, 1e-6, qo, go, ko,
                                                   position_base=4096 + i), stream, steps, warmup)
        nbytes = R * (ATT_H * 2 * ATT_D * 2 + ATT_KVH * ATT_D * 2 + 2 * ATT_H * ATT_D * 2 + ATT_KVH * ATT_D * 4)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[f"attn_prepare_rows{R}"] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                                        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
    return out


# ---------------------------------------------------------------------------
# Gated DeltaNet
# ---------------------------------------------------------------------------
def deltanet_legs(rt, dev, rng, steps, warmup):
    import torch
    import qm38
    c = DN
    ch = 2 * c["key_heads"] * c["key_head_dim"] + c["value_heads"] * c["value_head_dim"]
    VH, dv, dk = c["value_heads"], c["value_head_dim"], c["key_head_dim"]
    cfg = qm38.DnConfig(c["key_heads"], VH, dk, dv, c["conv_kernel_size"])
    w = rt.create_deltanet_weights(cfg, (rng.standard_normal((ch, 4)) * 0.5).astype(np.float32),
                                   np.zeros(VH, np.float32), np.zeros(VH, np.float32),
                                   (1 + 0.1 * rng.standard_normal(dv)).astype(np.float32))
    st = w.create_state()
    out = {}
    stream = torch.cuda.current_stream()
    for M in (1, 2048):
        qkv = torch.randn((M, ch), device=dev)
        z = torch.randn((M, VH * dv), device=dev)
        b = torch.randn((M, VH), device=dev)
        a = torch.randn((M, VH), device=dev)
        o = torch.empty((M, VH * dv), device=dev)
        if M == 1:
            fn = lambda i, m: rt.deltanet_step(w, st, qkv, z, b, a, 1e-6, o)
        else:
            fn = lambda i, m: rt.deltanet_prefill(w, st, qkv, z, b, a, M, 1e-6, o)
        ms, _ = timed(fn, stream, steps if M == 1 else max(2, steps // 10), warmup if M == 1 else 1)
        state = 2 * VH * dv * dk * 4 + 2 * ch * 3 * 4
        acts = M * (ch + VH * dv + 2 * VH + VH * dv) * 4
        gbs = (state + acts) / (ms * 1e-3) / 1e9
        key = "deltanet_step" if M == 1 else "deltanet_prefill_2048"
        out[key] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                    "tokens_per_s": round(M / (ms * 1e-3), 1)}
        if M > 1:
            # The recurrence's arithmetic (decay, S k, update, S q: 7 dk dv per
            # token and head), priced against the fp32 MFMA peak the chunked
            # scan runs on.
            tf = 7.0 * dk * dv * VH * M / (ms * 1e-3) / 1e12
            out[key].update({"TFLOP/s": round(tf, 2), "fp32_mfma_frac": round(tf / FP32_PEAK_TFLOPS, 4)})
    st.close()
    w.close()
    return out


def _dev_q4(rows: int, cols: int, gen, dev):
    """A random Q4 matrix made on the device (packed words, bf16 scales in
    [0.002, 0.012), biases -8 * scale)."""
    import torch
    import qm38
    w = torch.randint(-2 ** 31, 2 ** 31 - 1, (rows, cols // 8), dtype=torch.int32, device=dev, generator=gen)
    s = (torch.rand((rows, cols // 64), device=dev, generator=gen) * 0.01 + 0.002).to(torch.bfloat16)
    b = (-8 * s.float()).to(torch.bfloat16)
    return qm38.Runtime.job(w, s.view(torch.int16), b.view(torch.int16), rows)


def decode_graph_legs(rt, dev, rng, steps, warmup):
    """One token through a 4-layer block (3 DeltaNet + 1 full-attention layer,
    the 3:1 pattern of the hybrid model) at the BASELINE dimensions, eager
    (qm_decode_layers) and as HIP graph segments (qm_decode_graph)."""
    import torch
    import qm38
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    c = DN
    ch = 2 * c["key_heads"] * c["key_head_dim"] + c["value_heads"] * c["value_head_dim"]
    val = c["value_heads"] * c["value_head_dim"]
    keep, weight_bytes = [], 0
    kinds = ("linear", "linear", "linear", "full")

    def job(rows, cols):
        nonlocal weight_bytes
        weight_bytes += q4_bytes(rows, cols)
        return _dev_q4(rows, cols, gen, dev)

    def norm(n):
        t = (1 + 0.1 * torch.randn(n, device=dev, generator=gen)).float()
        keep.append(t)
        return t.data_ptr()

    layers = []
    for kind in kinds:
        L = dict(kind=kind, in_norm=norm(H), post_norm=norm(H), gate=job(I, H), up=job(I, H), down=job(H, I))
        if kind == "linear":
            L.update(qkv=job(ch, H), z=job(val, H), b=job(c["value_heads"], H), a=job(c["value_heads"], H),
                     out=job(H, val))
            cfg = qm38.DnConfig(c["key_heads"], c["value_heads"], c["key_head_dim"], c["value_head_dim"],
                                c["conv_kernel_size"])
            L["w"] = rt.create_deltanet_weights(cfg, (rng.standard_normal((ch, 4)) * 0.3).astype(np.float32),
                                                np.zeros(c["value_heads"], np.float32),
                                                np.zeros(c["value_heads"], np.float32),
                                                np.ones(c["value_head_dim"], np.float32))
        else:
            L.update(q=job(2 * ATT_H * ATT_D, H), k=job(ATT_KVH * ATT_D, H), v=job(ATT_KVH * ATT_D, H),
                     o=job(H, ATT_H * ATT_D), q_norm=norm(ATT_D), k_norm=norm(ATT_D))
        layers.append(L)
    rope = qm38.RopeConfig(ATT_D, 64, 1e7, 0, 0, 0)

    def request():
        alive, descs = [], []
        for L in layers:
            if L["kind"] == "linear":
                st = L["w"].create_state()
                alive.append(st)
                descs.append(qm38.DecodeLinearLayer(L["in_norm"], L["post_norm"], L["qkv"], L["z"], L["b"], L["a"],
                                                    L["out"], L["w"].handle.value, st.handle.value, L["gate"],
                                                    L["up"], L["down"]))
            else:
                kv = rt.create_q8_kv_state(ATT_KVH, ATT_D, 4096)
                alive.append(kv)
                descs.append(qm38.DecodeFullLayer(L["in_norm"], L["post_norm"], L["q"], L["k"], L["v"], L["o"],
                                                  L["q_norm"], L["k_norm"], ATT_H, rope, kv.handle.value, L["gate"],
                                                  L["up"], L["down"]))
        st = rt.create_decode_state(H)
        h0 = (rng.standard_normal(H) * 2).astype(np.float32)
        rt.lib.qm_copy_to_device(rt.handle, st.hidden_ptr, h0.ctypes.data, h0.nbytes)
        alive.append(st)
        return st, descs, alive

    stream = torch.cuda.current_stream()
    out = {}

    def host_us(fn, n=20):
        """Host time to enqueue one token (the GPU drains behind it)."""
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(n):
            fn(10_000 + i, None)
        t1 = time.perf_counter()
        torch.cuda.synchronize()
        return (t1 - t0) / n * 1e6

    st_e, descs_e, alive_e = request()
    eager = lambda i, m: rt.decode_layers(st_e, descs_e, (i, i, i), 1e-6)  # noqa: E731
    ms_e, _ = timed(eager, stream, steps, warmup)
    host_e = host_us(eager)
    st_g, descs_g, alive_g = request()
    graph = qm38.DecodeGraph(rt, st_g, descs_g, 1e-6)
    replay = lambda i, m: graph.run((i, i, i))  # noqa: E731
    ms_g, _ = timed(replay, stream, steps, warmup)
    host_g = host_us(replay)
    for key, ms, hu in (("decode_block4_eager", ms_e, host_e), ("decode_block4_graph", ms_g, host_g)):
        gbs = weight_bytes / (ms * 1e-3) / 1e9
        out[key] = {"us_per_token": round(ms * 1e3, 1), "host_enqueue_us_per_token": round(hu, 1),
                    "weight_bytes": weight_bytes, "GB/s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
    graph.close()
    for obj in alive_e + alive_g:
        obj.close()
    for L in layers:
        if "w" in L:
            L["w"].close()
    return out


# ---------------------------------------------------------------------------
# CPU baseline
# ---------------------------------------------------------------------------
def cpu_baseline_q4(seconds: float = 12.0):
    """Same decode-projection math (oracle/, fp32, OpenMP over rows) on host cores."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    from qm38 import synth
    rng = np.random.default_rng(99)
    w, s, b = synth.q4_matrix(rng, QKV, H)
    x = synth.bf16_normal(rng, (1, H))
    threads = min(os.cpu_count() or 1, int(os.environ.get("OMP_NUM_THREADS", "16") or 16))
    oracle.q4_project(x, w, s, b, threads=threads, fp32=True)  # warm
    n = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        oracle.q4_project(x, w, s, b, threads=threads, fp32=True)
        n += 1
    dt = time.perf_counter() - t0
    gbs = n * (q4_bytes(QKV, H) + 2 * H + 2 * QKV) / dt / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"QKV projection 5120->10240 (M=1) repeated {n}x over {dt:.1f}s, fp32 per-group "
                      f"accumulation (oracle qo_q4_project_f32)"}


def cpu_baseline_legs(seconds: float = 4.0):
    """The attention and DeltaNet legs' math on host cores (oracle/, OpenMP),
    each over a bounded sample, reported beside the GPU legs."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    rng = np.random.default_rng(98)
    threads = min(os.cpu_count() or 1, int(os.environ.get("OMP_NUM_THREADS", "16") or 16))
    out = {}

    def rate(fn):
        fn()
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds:
            fn()
            n += 1
        return (time.perf_counter() - t0) / n, n

    # Decode attention, one sequence at 32K (fp64-accumulated oracle, heads in parallel).
    T = 32768
    kq, ks = oracle.q8_quantize_rows(rng.standard_normal((T, ATT_KVH, ATT_D)).astype(np.float32))
    vq, vs = oracle.q8_quantize_rows(rng.standard_normal((T, ATT_KVH, ATT_D)).astype(np.float32))
    q = rng.standard_normal((1, ATT_H, ATT_D)).astype(np.float32)
    sec, n = rate(lambda: oracle.attention(q, q, kq, ks, vq, vs, T - 1, threads=threads))
    out["attn_decode_32k"] = {"us_per_token": round(sec * 1e6, 1),
                              "GB/s": round(attn_bytes(T) / sec / 1e9, 2), "cores": threads,
                              "sample": f"{n} decode tokens at T=32768, H=64 KVH=8 d=128 (qo_attention)"}
    # DeltaNet step and 2048-token prefill (fp32 oracle, value heads in parallel).
    c = DN
    ch = 2 * c["key_heads"] * c["key_head_dim"] + c["value_heads"] * c["value_head_dim"]
    VH, dv, dk = c["value_heads"], c["value_head_dim"], c["key_head_dim"]
    conv = (rng.standard_normal((ch, 4)) * 0.5).astype(np.float32)
    zero = np.zeros(VH, np.float32)
    norm = np.ones(dv, np.float32)
    for M, key in ((1, "deltanet_step"), (2048, "deltanet_prefill_2048")):
        acts = [rng.standard_normal(sh).astype(np.float32) for sh in ((M, ch), (M, VH * dv), (M, VH), (M, VH))]
        hist = np.zeros((ch, 3), np.float32)
        S = np.zeros((VH, dv, dk), np.float32)
        sec, n = rate(lambda: oracle.deltanet_prefill(c, conv, zero, zero, norm, *acts, 1e-6, hist, S))
        out[key] = {"us": round(sec * 1e6, 1), "tokens_per_s": round(M / sec, 1), "cores": threads,
                    "sample": f"{n} runs of {M} token(s), 16/32 heads, d=128 (qo_dn_prefill_f32)"}
    return out


def traffic_from_profiles():
    """HBM bytes per launch of the roofline kernel (the QKV + gate/up set), from
    the committed rocprofv3 FETCH_SIZE / WRITE_SIZE measurement (profiles/), or None."""
    p = ROOT / "profiles" / TRAFFIC_FILE
    try:
        return json.loads(p.read_text()).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


TRAFFIC_FILE = "q4_stream_qkv_gateup_traffic.json"
ROOF_KERNEL = "q4_stream_kernel"


def _counter_rows(d: str, counter: str):
    """(kernel name, KiB) per dispatch of `counter`, in dispatch order, from a rocprofv3 csv directory."""
    import csv
    import glob
    files = sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True))
    if not files:
        raise FileNotFoundError(f"no *counter_collection.csv under {d}")
    rows = []
    with open(files[0]) as f:
        for r in csv.DictReader(f):
            if r.get("Counter_Name") == counter:
                rows.append((int(r.get("Dispatch_Id", len(rows))), r["Kernel_Name"], float(r["Counter_Value"])))
    rows.sort()
    return [(k, v) for _, k, v in rows]


def traffic_summary(fetch_dir: str, write_dir: str) -> int:
    """HBM bytes per QKV + gate/up (M=1) set launch from FETCH_SIZE / WRITE_SIZE (KiB per dispatch), each
    scaled by what the same counter reads for a 256 MiB device copy of known size."""
    copy_bytes = 256 << 20
    out = {"kernel": None, "calibration": {"copy_bytes": copy_bytes}, "raw_KiB_per_dispatch": {}}
    per = {}
    for counter, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        rows = _counter_rows(d, counter)
        # The copy dispatches are the large non-q4 ones; the first (a small runtime copy) is excluded.
        copies = [v for k, v in rows if ROOF_KERNEL not in k and v * 1024 > copy_bytes / 4]
        q4 = [(k, v) for k, v in rows if ROOF_KERNEL in k]
        if not copies or not q4:
            raise RuntimeError(f"{counter}: expected copy and {ROOF_KERNEL} dispatches in {d}")
        factor = copy_bytes / (sum(copies) / len(copies) * 1024)
        out["calibration"][f"{counter}_KiB"] = round(sum(copies) / len(copies), 3)
        out["calibration"]["fetch_factor" if counter == "FETCH_SIZE" else "write_factor"] = round(factor, 4)
        out["raw_KiB_per_dispatch"][counter] = [v for _, v in q4]
        per[counter] = sum(v for _, v in q4) / len(q4) * 1024 * factor
        out["kernel"] = q4[0][0][:120] + " (QKV + gate/up SwiGLU set, M=1, 27B shapes)"
    alg = q4_bytes(QKV, H) + 2 * q4_bytes(I, H) + 2 * (H + QKV + I)
    out.update({"bytes_per_launch": int(per["FETCH_SIZE"] + per["WRITE_SIZE"]),
                "fetch_bytes": int(per["FETCH_SIZE"]), "write_bytes": int(per["WRITE_SIZE"]),
                "algorithmic_bytes": alg,
                "traffic_over_algorithmic": round((per["FETCH_SIZE"] + per["WRITE_SIZE"]) / alg, 4),
                "commands": [
                    "rocprofv3 --pmc FETCH_SIZE --kernel-trace -d prof_out/pmc_fetch -o fetch --output-format csv "
                    "-- python -u bench.py --traffic-probe",
                    "rocprofv3 --pmc WRITE_SIZE --kernel-trace -d prof_out/pmc_write -o write --output-format csv "
                    "-- python -u bench.py --traffic-probe",
                    "python bench.py --traffic-from prof_out/pmc_fetch prof_out/pmc_write"],
                "method": "per-dispatch counter (KiB) x (known copy bytes / the counter's reading for a 256 MiB "
                          "device copy); small copies excluded from the calibration mean"})
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", TRAFFIC_FILE)
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print(path)
    return 0


def gemm_counter_summary(d: str) -> int:
    """profiles/q4_gemm_gateup_m2048_counters.txt from a rocprofv3 --pmc run of
    bench.py --gemm-probe (per-dispatch SQ/GRBM counters of q4_gemm_kernel)."""
    rows = []
    for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        with open(f) as fh:
            rows += list(csv.DictReader(fh))
    per = {}
    for r in rows:
        if "q4_gemm_kernel" not in r["Kernel_Name"]:
            continue
        e = per.setdefault(int(r["Dispatch_Id"]), {"ns": int(r["End_Timestamp"]) - int(r["Start_Timestamp"])})
        e[r["Counter_Name"]] = float(r["Counter_Value"])
    if not per:
        print("no q4_gemm_kernel dispatches found", file=sys.stderr)
        return 1
    simds, cus, xcds = 1024, 256, 8
    lines = [
        "# rocprofv3 counters: q4_gemm_kernel, gate/up with SwiGLU, M = 2048 (BASELINE config 3)",
        "#",
        "# command (repo root, MI355X, one GPU):",
        "#   rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CYCLES SQ_BUSY_CU_CYCLES SQ_LDS_BANK_CONFLICT \\",
        "#     SQ_LDS_IDX_ACTIVE SQ_INSTS_LDS SQ_INSTS_MFMA SQ_WAIT_INST_LDS GRBM_GUI_ACTIVE --kernel-trace \\",
        "#     -d prof_out/gemm_pmc -o gemm --output-format csv -- python3 bench.py --gemm-probe",
        "#   python bench.py --gemm-counters-from prof_out/gemm_pmc",
        "#",
        "# GRBM_GUI_ACTIVE is summed over the 8 XCDs, so the kernel's GPU cycles are GRBM_GUI_ACTIVE / 8.",
        "# MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (cycles x 1024 SIMDs); each v_mfma_f32_32x32x16_f16 is",
        "# 32 busy cycles (SQ_INSTS_MFMA x 32 = SQ_VALU_MFMA_BUSY_CYCLES).  LDS active = SQ_LDS_IDX_ACTIVE /",
        "# (cycles x 256 CUs).  Durations run longer under counter collection than in the bench.",
        "",
        f"{'dispatch':>8} {'us':>9} {'GHz':>6} {'MFMA busy':>10} {'MFMA instr':>12} {'LDS active':>11} "
        f"{'LDS instr':>11} {'bank confl':>11}",
    ]
    for k in sorted(per):
        e = per[k]
        cyc = e.get("GRBM_GUI_ACTIVE", 0.0) / xcds
        if cyc <= 0:
            continue
        lines.append(f"{k:>8} {e['ns'] / 1e3:>9.1f} {cyc / e['ns']:>6.2f} "
                     f"{e.get('SQ_VALU_MFMA_BUSY_CYCLES', 0) / (cyc * simds):>10.1%} {e.get('SQ_INSTS_MFMA', 0):>12.0f} "
                     f"{e.get('SQ_LDS_IDX_ACTIVE', 0) / (cyc * cus):>11.1%} {e.get('SQ_INSTS_LDS', 0):>11.0f} "
                     f"{e.get('SQ_LDS_BANK_CONFLICT', 0):>11.0f}")
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "q4_gemm_gateup_m2048_counters.txt")
    with open(path, "w") as fh:
        fh.write("\n".join(lines) + "\n")
    print(path)
    return 0


def _short_kernel_name(name: str) -> str:
    n = name.replace("qm::(anonymous namespace)::", "").replace("(anonymous namespace)::", "")
    return n.replace("(qm::DecodeArgs)", "(DecodeArgs)").replace("(qm::GemmArgs)", "(GemmArgs)")


def stats_summary(prof_dir: str) -> int:
    """profiles/bench_all_legs_kernel_stats.txt from a rocprofv3 --kernel-trace --stats run of bench.py."""
    files = glob.glob(os.path.join(prof_dir, "**", "*kernel_stats.csv"), recursive=True)
    if not files:
        raise FileNotFoundError(f"no *kernel_stats.csv under {prof_dir}")
    with open(files[0]) as f:
        rows = list(csv.DictReader(f))
    lines = [
        "# rocprofv3 kernel statistics: bench.py (all legs, 20 timed steps)",
        "#",
        "# command (repo root, MI355X, one GPU):",
        "#   rocprofv3 --kernel-trace --stats -d prof_out/prof -o bench --output-format csv -- python3 -u bench.py "
        "--no-cpu --steps 20",
        "#   python bench.py --stats-from prof_out/prof",
        "#",
        "# Per-kernel averages mix the legs that launch the same template (q8_prefill_kernel<128,2> is the",
        "# causal prefill, including the 32K/128K cache fills of the attention legs; q4_gemm_kernel serves",
        "# M = 512 and 2048; q8_decode_kernel<128> serves the 32K single-sequence and ragged batch-8 legs).",
        "# The gate+up decode kernel (q4_decode_kernel<2, 1, true, true, true>, M = 1) is the bench's",
        "# roofline kernel.  bench.py's avg_launch_us for it comes from events around back-to-back",
        "# launches, so it also holds the gap between launches (about 1-2 us) and reads that much above",
        "# the kernel-only average here.",
        "",
        f"{'kernel':<100} {'calls':>6} {'avg_us':>10} {'min_us':>10} {'max_us':>10} {'pct':>7}",
    ]
    for r in sorted(rows, key=lambda r: -float(r["Percentage"])):
        lines.append(f"{_short_kernel_name(r['Name'])[:100]:<100} {int(r['Calls']):>6} "
                     f"{float(r['AverageNs']) / 1e3:>10.2f} {float(r['MinNs']) / 1e3:>10.2f} "
                     f"{float(r['MaxNs']) / 1e3:>10.2f} {float(r['Percentage']):>7.3f}")
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "bench_all_legs_kernel_stats.txt")
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")
    print(path)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--quick", action="store_true", help="headline only: no extra legs, no CPU baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--legs", default="decode,prefill,attn,deltanet,graph",
                    help="comma list of extra legs to run (the M=1 headline always runs)")
    ap.add_argument("--gemm-counters-from", metavar="PMC_DIR",
                    help="write profiles/q4_gemm_gateup_m2048_counters.txt from a --gemm-probe counter run")
    ap.add_argument("--gemm-probe", action="store_true",
                    help="only run six M=2048 gate/up GEMMs (for rocprofv3 --pmc passes)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="for rocprofv3 --pmc: 5 launches of a 256 MiB copy, then 5 gate+up M=1 launches")
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="turn the two --traffic-probe counter runs (rocprofv3 csv output directories) "
                         "into profiles/q4_stream_qkv_gateup_traffic.json (no GPU needed)")
    ap.add_argument("--stats-from", metavar="PROF_DIR",
                    help="turn a rocprofv3 --kernel-trace --stats run of bench.py into "
                         "profiles/bench_all_legs_kernel_stats.txt (no GPU needed)")
    args = ap.parse_args()
    if args.stats_from:
        return stats_summary(args.stats_from)
    if args.gemm_counters_from:
        return gemm_counter_summary(args.gemm_counters_from)
    if args.traffic_from:
        return traffic_summary(*args.traffic_from)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU mode (one GPU per box); "
              "run with --gpus 1", file=sys.stderr)
        return 2

    import torch
    import qm38
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    rt = qm38.Runtime(0)
    rt.set_stream(torch.cuda.current_stream())
    rng = np.random.default_rng(2026)

    log("[bench] uploading 3 weight copies")
    sets = q4_sets(rng, dev)
    if args.gemm_probe:
        # Six gate/up SwiGLU GEMMs at M = 2048, for
        # rocprofv3 --pmc passes over the prefill kernel.
        x = dev_array(synth_bf16(rng, (2048, H)), dev)
        h = torch.empty((2048, I), dtype=torch.int16, device=dev)
        for i in range(6):
            j = sets[i % NCOPY]
            rt.q4_swiglu(j["gate"][0], j["up"][0], x, H, 2048, h)
        torch.cuda.synchronize()
        rt.close()
        return 0
    if args.traffic_probe:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        x = dev_array(synth_bf16(rng, (1, H)), dev)
        h = torch.empty((1, I), dtype=torch.int16, device=dev)
        qo = torch.empty((1, QKV), dtype=torch.int16, device=dev)
        for i in range(5):
            dst.copy_(src)
        for i in range(5):
            j = sets[i % NCOPY]
            rt.q4_project_set([j["qkv"][0], j["gate"][0]], [None, j["up"][0]], x, H, 1, [qo, h])
        torch.cuda.synchronize()
        rt.close()
        return 0
    extras = {}
    head = None
    legs = set() if args.quick else set(args.legs.split(","))
    for M in (1, 4, 8) if "decode" in legs else (1,):
        log(f"[bench] q4 decode set M={M}")
        ms, kern, wb, ab, _ = q4_leg(rt, dev, sets, M, rng, args.steps, args.warmup)
        step_bytes = sum(wb.values()) + sum(ab.values())
        gbs = step_bytes / (ms * 1e-3) / 1e9
        extras[f"q4_decode_set_M{M}"] = {
            "GB/s": round(gbs, 1), "ms_per_step": round(ms, 4), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "kernel_us": {k: round(v * 1e3, 2) for k, v in kern.items()},
            "kernel_hbm_frac": {k: round((wb[k] + ab[k]) / (kern[k] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4) for k in kern}}
        if M == 1:
            head = (gbs, ms, step_bytes, wb["qkv_gateup"] + ab["qkv_gateup"], kern["qkv_gateup"])
            p10, p50, p90 = step_distribution(q4_leg.last_step, torch.cuda.current_stream(), max(args.steps, 100))
            extras["q4_decode_set_M1"]["step_us_p10_p50_p90"] = [p10, p50, p90]
    if "decode" in legs:
        log("[bench] q4 matvec 4096x4096 (config 1)")
        extras["q4_matvec_4096_M1"] = matvec_4096_leg(rt, dev, rng, args.steps, args.warmup)
    if "prefill" in legs:
        for M in (512, 2048):
            log(f"[bench] q4 prefill GEMM set M={M}")
            steps = max(3, args.steps // 10)
            ms, kern, wb, ab, fl = q4_leg(rt, dev, sets, M, rng, steps, 2)
            tf = sum(fl.values()) / (ms * 1e-3) / 1e12
            extras[f"q4_prefill_set_M{M}"] = {
                "TFLOP/s": round(tf, 1), "ms_per_step": round(ms, 3), "mfma_frac": round(tf / MFMA_PEAK_TFLOPS, 4),
                "kernel_us": {k: round(v * 1e3, 1) for k, v in kern.items()},
                "kernel_TFLOP/s": {k: round(fl[k] / (kern[k] * 1e-3) / 1e12, 1) for k in kern}}
    del sets
    torch.cuda.empty_cache()
    if "attn" in legs:
        log("[bench] attention")
        extras.update(attention_legs(rt, dev, rng, args.steps, args.warmup))
    if "deltanet" in legs:
        log("[bench] deltanet")
        extras.update(deltanet_legs(rt, dev, rng, args.steps, args.warmup))
    if "graph" in legs:
        log("[bench] decode graph")
        extras.update(decode_graph_legs(rt, dev, rng, args.steps, args.warmup))

    gbs, ms, step_bytes, gu_bytes, gu_ms = head
    gu_achieved = gu_bytes / (gu_ms * 1e-3) / 1e9
    result = {
        "metric": "Q4 matvec GB/s (% HBM peak); Q8-KV attn us/token @32K; prefill TFLOP/s",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4-affine weights x bf16 activations, fp32 accumulate",
        "data": "synthetic (seeded; BASELINE config distributions; 3 rotating weight copies)",
        "config": {"workload": "BASELINE config 2: Q4 decode projection set, QKV 5120->10240, gate+up "
                               "5120->2x17408 (+SwiGLU), down 17408->5120, M=1",
                   "step_bytes": step_bytes, "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(gu_achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_achieved / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles(),
                     "kernel": "q4_stream_kernel (QKV + gate/up pairs with SwiGLU in one launch, M=1)",
                     "bytes_per_launch": gu_bytes, "avg_launch_us": round(gu_ms * 1e3, 2)},
        "extras": extras,
    }
    if not args.no_cpu and not args.quick:
        log("[bench] cpu baseline")
        result["cpu_baseline"] = cpu_baseline_q4()
        if legs & {"attn", "deltanet"}:
            log("[bench] cpu baselines of the attention / DeltaNet legs")
            result["extras"]["cpu_legs"] = cpu_baseline_legs()
    else:
        result["cpu_baseline"] = None
    rt.close()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
