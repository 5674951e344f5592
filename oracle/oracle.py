"""ctypes front-end of the CPU oracle (oracle/qm_oracle.cpp).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg.  The product never imports it.  Also holds the
pure-Python restatement of the reference's LogicalPageTable
(/root/reference/src/paged_kv.rs:12-98), which is small integer logic.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        vp, u32, i32 = C.c_void_p, C.c_uint32, C.c_int
        L.qo_bf16_to_f32.argtypes = [C.c_uint16]
        L.qo_bf16_to_f32.restype = C.c_float
        L.qo_f32_to_bf16.argtypes = [C.c_float]
        L.qo_f32_to_bf16.restype = C.c_uint16
        for n in ("qo_q4_project", "qo_q4_project_f32"):
            getattr(L, n).argtypes = [vp, u32, u32, vp, vp, vp, u32, vp, i32]
            getattr(L, n).restype = None
        L.qo_swiglu.argtypes = [vp, vp, C.c_size_t, vp]
        L.qo_q8_quantize.argtypes = [vp, u32, vp, vp]
        L.qo_q8_quantize_rows.argtypes = [vp, C.c_uint64, u32, vp, vp]
        L.qo_attention.argtypes = [vp, vp, vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, vp, i32]
        for n in ("qo_dn_prefill_f32", "qo_dn_prefill_f64"):
            getattr(L, n).argtypes = [u32, u32, u32, u32, u32, vp, vp, vp, vp, vp, vp, vp, vp, u32,
                                      C.c_float, vp, vp, vp]
        L.qo_attn_prepare.argtypes = [vp, vp, vp, vp, u32, u32, u32, u32, u32, C.c_double, u32, u32, u32, vp, u32,
                                      C.c_float, vp, vp, vp]
        L.qo_residual_rmsnorm.argtypes = [vp, vp, vp, u32, u32, C.c_float, vp]
        L.qo_num_threads.restype = i32
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data if a is not None else None


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def q4_project(x_bf16, packed, scales, biases, threads: int = 0, fp32: bool = False) -> np.ndarray:
    """y fp32 [M][N] for x bf16 [M][K] (double accumulation unless fp32=True)."""
    x = _c(x_bf16, np.uint16)
    if x.ndim == 1:
        x = x[None]
    M, K = x.shape
    w = _c(packed, np.uint32)
    N = w.shape[0]
    s = _c(scales, np.uint16)
    b = _c(biases, np.uint16)
    y = np.zeros((M, N), np.float32)
    fn = lib().qo_q4_project_f32 if fp32 else lib().qo_q4_project
    fn(_p(x), M, K, _p(w), _p(s), _p(b), N, _p(y), threads)
    return y


def swiglu(g, u) -> np.ndarray:
    g = _c(g, np.float32)
    u = _c(u, np.float32)
    h = np.zeros_like(g)
    lib().qo_swiglu(_p(g), _p(u), g.size, _p(h))
    return h


def q8_quantize(x) -> tuple[np.ndarray, np.float32]:
    x = _c(x, np.float32)
    q = np.zeros(x.shape, np.int8)
    s = np.zeros(1, np.float32)
    lib().qo_q8_quantize(_p(x), x.size, _p(q), _p(s))
    return q, s[0]


def q8_quantize_rows(x) -> tuple[np.ndarray, np.ndarray]:
    """x fp32 [..., d] -> (int8 [..., d], fp32 scales [...])."""
    x = _c(x, np.float32)
    flat = x.reshape(-1, x.shape[-1])
    q = np.zeros(flat.shape, np.int8)
    s = np.zeros(flat.shape[0], np.float32)
    if flat.shape[0]:
        lib().qo_q8_quantize_rows(_p(flat), flat.shape[0], flat.shape[1], _p(q), _p(s))
    return q.reshape(x.shape), s.reshape(x.shape[:-1])


def attention(q, gate, keys, kscale, values, vscale, start: int, threads: int = 0) -> np.ndarray:
    """q fp32 [rows][H][d]; cache token-major [T][KVH][d]; returns fp32 [rows][H][d]."""
    q = _c(q, np.float32)
    rows, H, d = q.shape
    keys = _c(keys, np.int8)
    T, KVH, _ = keys.shape
    g = _c(gate, np.float32) if gate is not None else None
    o = np.zeros_like(q)
    lib().qo_attention(_p(q), _p(g), _p(keys), _p(_c(kscale, np.float32)), _p(_c(values, np.int8)),
                       _p(_c(vscale, np.float32)), rows, H, KVH, d, start, T, _p(o), threads)
    return o


def deltanet_prefill(cfg: dict, conv_w, a_log, dt_bias, norm, qkv, z, b, a, eps, hist, S,
                     f64: bool = False):
    """Sequential DeltaNet over M tokens.  Returns (out [M][VH*dv], hist, S) (copies)."""
    KH, VH, dk, dv, ks = (cfg[k] for k in ("key_heads", "value_heads", "key_head_dim", "value_head_dim",
                                           "conv_kernel_size"))
    qkv = _c(qkv, np.float32)
    M = qkv.shape[0]
    dt = np.float64 if f64 else np.float32
    hist = np.array(hist, dtype=dt, copy=True)
    S = np.array(S, dtype=dt, copy=True)
    if hist.size == 0:
        hist = np.zeros(1, dt)
    out = np.zeros((M, VH * dv), np.float32)
    fn = lib().qo_dn_prefill_f64 if f64 else lib().qo_dn_prefill_f32
    fn(KH, VH, dk, dv, ks, _p(_c(conv_w, np.float32)), _p(_c(a_log, np.float32)), _p(_c(dt_bias, np.float32)),
       _p(_c(norm, np.float32)), _p(qkv), _p(_c(z, np.float32)), _p(_c(b, np.float32)), _p(_c(a, np.float32)),
       M, eps, _p(hist), _p(S), _p(out))
    return out, hist, S


class PageTableError(Exception):
    pass


class LogicalPageTable:
    """Restatement of LogicalPageTable (paged_kv.rs:12-98)."""

    def __init__(self, max_tokens: int, page_tokens: int):
        if max_tokens == 0 or page_tokens == 0:
            raise PageTableError("ZeroCapacity")
        self.max_tokens = max_tokens
        self.page_tokens = page_tokens
        self.sequence_tokens = 0
        self.pages = [None] * (-(-max_tokens // page_tokens))
        self.next_page_id = 0

    def append(self, n: int):
        if n == 0:
            raise PageTableError("EmptyAppend")
        start = self.sequence_tokens
        end = start + n
        if end > self.max_tokens:
            raise PageTableError("CapacityExceeded")
        first, last = start // self.page_tokens, (end - 1) // self.page_tokens
        for p in range(first, last + 1):
            if self.pages[p] is None:
                self.pages[p] = self.next_page_id
                self.next_page_id += 1
        self.sequence_tokens = end
        return (start, end, first, last)

    def allocated_pages(self) -> int:
        return sum(p is not None for p in self.pages)

    def page_for_token(self, token: int):
        if token >= self.sequence_tokens:
            return None
        return self.pages[token // self.page_tokens]


def attn_prepare(q_with_gate, k, q_norm, k_norm, head_dim: int, rotary_dim: int, theta: float, eps: float,
                 sections=None, positions=None, base: int = 0):
    """Full-attention q/k preparation (qo_attn_prepare).  q_with_gate fp32
    [M][H][2 hd], k fp32 [M][KVH][hd]; sections (s1, s2) or None; positions
    uint32 [3][M] or None (every axis = base + row).  Returns (q, gate, k) fp32."""
    qg = _c(q_with_gate, np.float32)
    kk = _c(k, np.float32)
    M, H = qg.shape[0], qg.shape[1]
    KVH = kk.shape[1]
    q = np.zeros((M, H, head_dim), np.float32)
    g = np.zeros((M, H, head_dim), np.float32)
    ko = np.zeros((M, KVH, head_dim), np.float32)
    pos = None if positions is None else _c(positions, np.uint32)
    s1, s2 = sections if sections is not None else (0, 0)
    lib().qo_attn_prepare(_p(qg), _p(kk), _p(_c(q_norm, np.float32)), _p(_c(k_norm, np.float32)), M, H, KVH,
                          head_dim, rotary_dim, float(theta), s1, s2, int(sections is not None), _p(pos), base, eps,
                          _p(q), _p(g), _p(ko))
    return q, g, ko


def residual_rmsnorm(hidden, w, eps: float, delta=None):
    """qo_residual_rmsnorm: returns (hidden + delta in fp32, fp64 RMSNorm(hidden) * w).
    hidden fp32 [M][n] (not modified), delta fp32 [M][n] or None, w fp32 [n]."""
    h = np.array(hidden, dtype=np.float32, copy=True)
    if h.ndim == 1:
        h = h[None]
    M, n = h.shape
    out = np.zeros((M, n), np.float64)
    d = _c(np.reshape(delta, (M, n)), np.float32) if delta is not None else None
    lib().qo_residual_rmsnorm(_p(h), _p(d), _p(_c(w, np.float32)), M, n, eps, _p(out))
    return h, out
