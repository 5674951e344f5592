"""qm38 benchmark: the reference's per-token compute path on one MI355X.

Headline (`value`): MLX affine-Q4 decode projection set at 27B-class shapes
with one activation row: fused QKV 5120->10240, gate+up
5120->2x17408 with SwiGLU in the epilogue, down 17408->5120.  One step = one
pass of the three projections; `value` = algorithmic bytes of the step / step
time (GB/s), inputs resident in HBM.  Three copies of the weights (540 MB)
rotate between steps so the 256 MB MALL cannot serve them.

`extras` carries the other legs of the metric, each against its roofline:
the decode set at 2, 4 and 8 rows; Q8-KV decode attention at 32K context
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


# Leg markers for per-leg kernel statistics: with --markers <file>, every
# timed region starts and ends with a tiny torch sleep kernel ("spin_kernel"
# in a rocprofv3 kernel trace) and its label is appended to <file>;
# `--stats-from` then assigns each dispatch to the region around it.
_MARKERS = None


def leg_marker(label: str) -> None:
    if not _MARKERS:
        return
    import torch
    torch.cuda._sleep(1)
    with open(_MARKERS, "a") as f:
        f.write(label + "\n")


def timed(step, stream, steps: int, warmup: int, label: str = "other"):
    """Runs warmup + steps calls of step(i, marks); returns (ms per step, per-step mark lists)."""
    import torch
    ev = Events(stream)
    leg_marker(label)
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
    leg_marker("-")
    return t0.elapsed_time(t1) / steps, marks_all


def step_distribution(step, stream, steps: int, warmup: int = 2, label: str = "other"):
    """Per-step times (us) from one event after each step: (p10, median, p90).
    The events sit between steps, so the set's own kernels stay back to back."""
    import torch
    ev = Events(stream)
    leg_marker(label)
    for i in range(warmup):
        step(i, None)
    torch.cuda.synchronize()
    gpu_blocker()
    marks = [ev.mark()]
    for i in range(steps):
        step(warmup + i, None)
        marks.append(ev.mark())
    torch.cuda.synchronize()
    leg_marker("-")
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
    ms, _ = timed(step, stream, steps, warmup, f"q4_set_M{M}")
    # Per-kernel durations: each projection alone, back to back (events only
    # around the whole run, so no event sits between the timed kernels).
    calls = {
        "qkv_gateup": lambda i, m: qkv_gateup(sets[i % NCOPY]),
        "down": lambda i, m: rt.q4_project([sets[i % NCOPY]["down"][0]], h, I, M, [y]),
    }
    per = [timed(fn, stream, steps, 2, f"q4_set_M{M}:{name}")[0] for name, fn in calls.items()]
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
                  warmup, "q4_matvec_4096")
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
    ms, _ = timed(lambda i, m: rt.gqa_attention_q8([caches[i % NC]], q, g, k, v, ATT_H, o), stream, steps, warmup,
                  "attn_decode_32k")
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
    ms, _ = timed(lambda i, m: rt.gqa_attention_q8(caches, q, g, k, v, ATT_H, o), stream, steps, warmup,
                  "attn_decode_ragged_b8")
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
    ms, _ = timed(lambda i, m: rt.gqa_attention_q8_prefill(caches[i], q, g, k, v, ATT_H, P, o), stream, reps, 1,
                  "attn_prefill_2048_on_4k")
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
                                                   position_base=4096 + i), stream, steps, warmup,
                      f"attn_prepare_rows{R}")
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
        ms, _ = timed(fn, stream, steps if M == 1 else max(2, steps // 10), warmup if M == 1 else 1,
                      "deltanet_step" if M == 1 else "deltanet_prefill_2048")
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
    ms_e, _ = timed(eager, stream, steps, warmup, "decode_block4_eager")
    host_e = host_us(eager)
    st_g, descs_g, alive_g = request()
    graph = qm38.DecodeGraph(rt, st_g, descs_g, 1e-6)
    replay = lambda i, m: graph.run((i, i, i))  # noqa: E731
    ms_g, _ = timed(replay, stream, steps, warmup, "decode_block4_graph")
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


# HBM traffic probes: each leg's setup, then five 256 MiB device copies (the
# counters' calibration), then `calls` launches of the leg; rocprofv3 --pmc
# FETCH_SIZE and WRITE_SIZE runs of `bench.py --traffic-probe LEG` give each
# dispatch's KiB, and `--traffic-from` turns them into bytes per call.
PROBE_CALLS = 5
PROBE_FILES = {
    "q4_set": TRAFFIC_FILE,
    "q4_set_m4": "q4_mma_qkv_gateup_m4_traffic.json",
    "attn_decode_32k": "q8_decode_attn_32k_traffic.json",
    "attn_prefill_2048": "q8_prefill_attn_2048_on_4k_traffic.json",
    "deltanet_step": "dn_step_traffic.json",
    "deltanet_prefill_2048": "dn_prefill_2048_traffic.json",
}


def probe_alg_bytes(leg: str) -> int:
    """Algorithmic HBM bytes of one call of a probed leg."""
    VH, dv, dk = DN["value_heads"], DN["value_head_dim"], DN["key_head_dim"]
    ch = 2 * DN["key_heads"] * dk + VH * dv
    if leg in ("q4_set", "q4_set_m4"):
        M = 4 if leg == "q4_set_m4" else 1
        return q4_bytes(QKV, H) + 2 * q4_bytes(I, H) + 2 * M * (H + QKV + I)
    if leg == "attn_decode_32k":
        # the cache read at T = 32768 + 1, q / gate in, output and the appended row
        return attn_bytes(32769) + 3 * ATT_H * ATT_D * 2 + ATT_KVH * (2 * ATT_D + 8)
    if leg == "attn_prefill_2048":
        P, T = 2048, 4096
        return attn_bytes(T + P) + P * (3 * ATT_H * ATT_D * 2 + 2 * ATT_KVH * ATT_D * 4)
    M = 1 if leg == "deltanet_step" else 2048
    return 2 * VH * dv * dk * 4 + 2 * ch * 3 * 4 + M * (ch + VH * dv + 2 * VH + VH * dv) * 4
    

def traffic_probe(rt, dev, rng, sets, leg: str) -> None:
    """Setup, calibration copies, then PROBE_CALLS calls of `leg` (for rocprofv3 --pmc)."""
    import torch
    from qm38 import synth
    if leg in ("q4_set", "q4_set_m4"):
        M = 4 if leg == "q4_set_m4" else 1  # M = 4: the MFMA streaming kernel
        x = dev_array(synth_bf16(rng, (M, H)), dev)
        h = torch.empty((M, I), dtype=torch.int16, device=dev)
        qo = torch.empty((M, QKV), dtype=torch.int16, device=dev)
        call = lambda i: rt.q4_project_set([sets[i % NCOPY]["qkv"][0], sets[i % NCOPY]["gate"][0]],  # noqa: E731
                                           [None, sets[i % NCOPY]["up"][0]], x, H, M, [qo, h])
    elif leg == "attn_decode_32k":
        caches = []
        for _ in range(PROBE_CALLS):
            c = kv_cache(rt, 32768 + 8)
            kv_fill(rt, dev, c, rng, 32768)
            caches.append(c)
        q = dev_array(synth.bf16_normal(rng, (1, ATT_H, ATT_D)), dev)
        g = dev_array(synth.bf16_normal(rng, (1, ATT_H, ATT_D)), dev)
        k = torch.randn((1, ATT_KVH, ATT_D), dtype=torch.float32, device=dev)
        o = torch.empty((1, ATT_H, ATT_D), dtype=torch.int16, device=dev)
        call = lambda i: rt.gqa_attention_q8([caches[i]], q, g, k, k, ATT_H, o)  # noqa: E731
    elif leg == "attn_prefill_2048":
        P, T = 2048, 4096
        caches = [kv_cache(rt, T + P) for _ in range(PROBE_CALLS)]
        for c in caches:
            kv_fill(rt, dev, c, rng, T)
        q = dev_array(synth.bf16_normal(rng, (P, ATT_H, ATT_D)), dev)
        g = dev_array(synth.bf16_normal(rng, (P, ATT_H, ATT_D)), dev)
        k = torch.randn((P, ATT_KVH, ATT_D), dtype=torch.float32, device=dev)
        o = torch.empty((P, ATT_H, ATT_D), dtype=torch.int16, device=dev)
        call = lambda i: rt.gqa_attention_q8_prefill(caches[i], q, g, k, k, ATT_H, P, o)  # noqa: E731
    else:
        import qm38
        VH, dv, dk = DN["value_heads"], DN["value_head_dim"], DN["key_head_dim"]
        ch = 2 * DN["key_heads"] * dk + VH * dv
        cfg = qm38.DnConfig(DN["key_heads"], VH, dk, dv, DN["conv_kernel_size"])
        w = rt.create_deltanet_weights(cfg, (rng.standard_normal((ch, 4)) * 0.5).astype(np.float32),
                                       np.zeros(VH, np.float32), np.zeros(VH, np.float32),
                                       np.ones(dv, np.float32))
        st = w.create_state()
        M = 1 if leg == "deltanet_step" else 2048
        qkv, z = torch.randn((M, ch), device=dev), torch.randn((M, VH * dv), device=dev)
        b, a = torch.randn((M, VH), device=dev), torch.randn((M, VH), device=dev)
        o = torch.empty((M, VH * dv), device=dev)
        if M == 1:
            call = lambda i: rt.deltanet_step(w, st, qkv, z, b, a, 1e-6, o)  # noqa: E731
        else:
            call = lambda i: rt.deltanet_prefill(w, st, qkv, z, b, a, M, 1e-6, o)  # noqa: E731
    torch.cuda.synchronize()
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    for i in range(PROBE_CALLS):
        call(i)
    torch.cuda.synchronize()


def traffic_summary(leg: str, fetch_dir: str, write_dir: str) -> int:
    """HBM bytes per call of a probed leg from FETCH_SIZE / WRITE_SIZE (KiB per dispatch), each scaled by
    what the same counter reads for a 256 MiB device copy of known size."""
    copy_bytes = 256 << 20
    out = {"leg": leg, "calibration": {"copy_bytes": copy_bytes}, "kernels": {}}
    per = {}
    for counter, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        rows = _counter_rows(d, counter)
        big = [i for i, (k, v) in enumerate(rows) if v * 1024 > copy_bytes / 4 and "copy" in k.lower()]
        if len(big) < 5:
            raise RuntimeError(f"{counter}: expected 5 calibration copies in {d}")
        copies = [rows[i][1] for i in big[-5:]]
        factor = copy_bytes / (sum(copies) / len(copies) * 1024)
        out["calibration"][f"{counter}_KiB"] = round(sum(copies) / len(copies), 3)
        out["calibration"]["fetch_factor" if counter == "FETCH_SIZE" else "write_factor"] = round(factor, 4)
        after = rows[big[-1] + 1:]  # the leg's calls
        for k, v in after:
            name = _short_kernel_name(k)[:120]
            e = out["kernels"].setdefault(name, {})
            e.setdefault(counter, []).append(v)
        per[counter] = sum(v for _, v in after) * 1024 * factor / PROBE_CALLS
    for e in out["kernels"].values():
        n = max(len(e.get("FETCH_SIZE", [])), 1)
        e["dispatches_per_call"] = n / PROBE_CALLS
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            f = out["calibration"]["fetch_factor" if counter == "FETCH_SIZE" else "write_factor"]
            e[counter.lower().replace("_size", "_bytes_per_call")] = int(sum(e.pop(counter, [])) * 1024 * f
                                                                         / PROBE_CALLS)
    alg = probe_alg_bytes(leg)
    out.update({"bytes_per_launch" if leg == "q4_set" else "bytes_per_call": int(per["FETCH_SIZE"] + per["WRITE_SIZE"]),
                "fetch_bytes": int(per["FETCH_SIZE"]), "write_bytes": int(per["WRITE_SIZE"]),
                "algorithmic_bytes": alg,
                "traffic_over_algorithmic": round((per["FETCH_SIZE"] + per["WRITE_SIZE"]) / alg, 4),
                "commands": [
                    f"rocprofv3 --pmc FETCH_SIZE --kernel-trace -d prof_out/f_{leg} -o fetch --output-format csv "
                    f"-- python -u bench.py --traffic-probe {leg}",
                    f"rocprofv3 --pmc WRITE_SIZE --kernel-trace -d prof_out/w_{leg} -o write --output-format csv "
                    f"-- python -u bench.py --traffic-probe {leg}",
                    f"python bench.py --traffic-from {leg} prof_out/f_{leg} prof_out/w_{leg}"],
                "method": f"per-dispatch counter (KiB) x (known copy bytes / the counter's reading for a 256 MiB "
                          f"device copy), summed over the {PROBE_CALLS} calls after the copies and divided by "
                          f"{PROBE_CALLS}"})
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", PROBE_FILES[leg])
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print(path)
    return 0


GEMM_PROBES = {"gateup_m2048": "gate/up with SwiGLU, M = 2048", "qkv_m512": "QKV 5120 -> 10240, M = 512"}


def gemm_counter_summary(shape: str, d: str) -> int:
    """profiles/q4_gemm_<shape>_counters.txt from a rocprofv3 --pmc run of
    bench.py --gemm-probe <shape> (per-dispatch SQ/GRBM counters of q4_gemm_kernel)."""
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
        f"# rocprofv3 counters: q4_gemm_kernel, {GEMM_PROBES[shape]} (BASELINE config 3)",
        "#",
        "# command (repo root, MI355X, one GPU):",
        "#   rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CYCLES SQ_BUSY_CU_CYCLES SQ_LDS_BANK_CONFLICT \\",
        "#     SQ_LDS_IDX_ACTIVE SQ_INSTS_LDS SQ_INSTS_MFMA SQ_WAIT_INST_LDS GRBM_GUI_ACTIVE --kernel-trace \\",
        f"#     -d prof_out/gemm_pmc -o gemm --output-format csv -- python3 bench.py --gemm-probe {shape}",
        f"#   python bench.py --gemm-counters-from {shape} prof_out/gemm_pmc",
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
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"q4_gemm_{shape}_counters.txt")
    with open(path, "w") as fh:
        fh.write("\n".join(lines) + "\n")
    print(path)
    return 0


def _short_kernel_name(name: str) -> str:
    n = name.replace("qm::(anonymous namespace)::", "").replace("(anonymous namespace)::", "")
    return n.replace("(qm::DecodeArgs)", "(DecodeArgs)").replace("(qm::GemmArgs)", "(GemmArgs)")


def stats_summary(prof_dir: str) -> int:
    """profiles/bench_kernel_stats_by_leg.txt from a rocprofv3 --kernel-trace run of
    bench.py --markers <prof_dir>/legs.txt: per timed region (warmup included),
    each kernel's calls and durations."""
    files = glob.glob(os.path.join(prof_dir, "**", "*kernel_trace.csv"), recursive=True)
    if not files:
        raise FileNotFoundError(f"no *kernel_trace.csv under {prof_dir}")
    with open(os.path.join(prof_dir, "legs.txt")) as f:
        labels = [ln.strip() for ln in f if ln.strip()]
    with open(files[0]) as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    per, order, cur, li, filler = {}, [], None, 0, 0
    for r in rows:
        name = r["Kernel_Name"]
        if "spin_kernel" in name:
            if li >= len(labels):
                raise ValueError("more marker kernels than labels")
            cur = None if labels[li] == "-" else labels[li]
            li += 1
            if cur is not None and cur not in per:
                per[cur] = {}
                order.append(cur)
            continue
        if cur is None:
            continue
        if name.startswith("Cijk_"):  # the fp16 GEMMs that keep the GPU busy while steps are enqueued
            filler += 1
            continue
        ns = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        per[cur].setdefault(_short_kernel_name(name), []).append(ns)
    lines = [
        "# rocprofv3 kernel statistics per bench.py leg (each timed region, warmup included)",
        "#",
        "# command (repo root, MI355X, one GPU):",
        "#   rocprofv3 --kernel-trace -d prof_out/legs -o bench --output-format csv -- python3 -u bench.py "
        "--no-cpu --steps 20 --markers prof_out/legs/legs.txt",
        "#   python bench.py --stats-from prof_out/legs",
        "#",
        "# Regions are delimited by marker kernels (torch's sleep kernel) that bench.py launches around each",
        "# timed region; setup work between regions (uploads, cache fills) is left out, and so are the fp16",
        f"# GEMMs that keep the GPU busy while a region's steps are enqueued ({filler} dispatches).",
        "# q4_set_M1:qkv_gateup / :down time each launch of the headline set alone; q4_set_M1 is the set.",
    ]
    for leg in order:
        lines += ["", f"[{leg}]", f"  {'kernel':<92} {'calls':>6} {'avg_us':>9} {'min_us':>9} {'max_us':>9}"]
        for k, v in sorted(per[leg].items(), key=lambda kv: -sum(kv[1])):
            a = np.array(v) / 1e3
            lines.append(f"  {k[:92]:<92} {len(a):>6} {a.mean():>9.2f} {a.min():>9.2f} {a.max():>9.2f}")
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "bench_kernel_stats_by_leg.txt")
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
    ap.add_argument("--gemm-counters-from", nargs=2, metavar=("SHAPE", "PMC_DIR"),
                    help="write profiles/q4_gemm_<SHAPE>_counters.txt from a --gemm-probe counter run")
    ap.add_argument("--gemm-probe", nargs="?", const="gateup_m2048", choices=sorted(GEMM_PROBES), metavar="SHAPE",
                    help="only run six prefill GEMMs of SHAPE (for rocprofv3 --pmc passes)")
    ap.add_argument("--traffic-probe", nargs="?", const="q4_set", choices=sorted(PROBE_FILES), metavar="LEG",
                    help="for rocprofv3 --pmc: the leg's setup, 5 launches of a 256 MiB copy, then 5 calls of "
                         "the leg (default q4_set: the QKV + gate/up set at M=1)")
    ap.add_argument("--traffic-from", nargs=3, metavar=("LEG", "FETCH_DIR", "WRITE_DIR"),
                    help="turn the two --traffic-probe counter runs of LEG (rocprofv3 csv output directories) "
                         "into its profiles/*_traffic.json (no GPU needed)")
    ap.add_argument("--stats-from", metavar="PROF_DIR",
                    help="turn a rocprofv3 --kernel-trace run of bench.py --markers PROF_DIR/legs.txt into "
                         "profiles/bench_kernel_stats_by_leg.txt (no GPU needed)")
    ap.add_argument("--markers", metavar="FILE",
                    help="launch a marker kernel around each timed region and list the regions in FILE")
    args = ap.parse_args()
    global _MARKERS
    if args.markers:
        _MARKERS = args.markers
        open(args.markers, "w").close()
    if args.stats_from:
        return stats_summary(args.stats_from)
    if args.gemm_counters_from:
        return gemm_counter_summary(*args.gemm_counters_from)
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
    sets = q4_sets(rng, dev) if args.traffic_probe in (None, "q4_set", "q4_set_m4") else None
    if args.gemm_probe:
        # Six GEMMs of one BASELINE config 3 shape, for rocprofv3 --pmc
        # passes over the prefill kernel.
        M = 2048 if args.gemm_probe == "gateup_m2048" else 512
        x = dev_array(synth_bf16(rng, (M, H)), dev)
        h = torch.empty((M, I), dtype=torch.int16, device=dev)
        qo = torch.empty((M, QKV), dtype=torch.int16, device=dev)
        for i in range(6):
            j = sets[i % NCOPY]
            if M == 2048:
                rt.q4_swiglu(j["gate"][0], j["up"][0], x, H, M, h)
            else:
                rt.q4_project([j["qkv"][0]], x, H, M, [qo])
        torch.cuda.synchronize()
        rt.close()
        return 0
    if args.traffic_probe:
        traffic_probe(rt, dev, rng, sets, args.traffic_probe)
        rt.close()
        return 0
    extras = {}
    head = None
    legs = set() if args.quick else set(args.legs.split(","))
    for M in (1, 2, 4, 8) if "decode" in legs else (1,):
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
            p10, p50, p90 = step_distribution(q4_leg.last_step, torch.cuda.current_stream(), max(args.steps, 100),
                                              label="q4_set_M1:distribution")
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
