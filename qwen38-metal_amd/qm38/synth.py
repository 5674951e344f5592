"""Seeded synthetic inputs with the distributions of the benchmark configs.

Q4 weights: nibbles uniform 0..15 (uniform u32 words have i.i.d. uniform
nibbles), bf16 scales ~ U(0.005, 0.02), bf16 biases = -8*scale + N(0, 1e-3);
activations bf16 N(0, 1).  All generators take a numpy Generator so that CPU
checks and GPU runs see identical bytes.
"""
from __future__ import annotations

import numpy as np


def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bits (qwen38.metal:22-26)."""
    bits = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def q4_matrix(rng: np.random.Generator, rows: int, cols: int):
    """Returns (packed u32 [rows][cols/8], scales bf16 [rows][cols/64], biases bf16)."""
    assert cols % 64 == 0
    packed = rng.integers(0, 2**32, size=(rows, cols // 8), dtype=np.uint64).astype(np.uint32)
    scale = rng.uniform(0.005, 0.02, size=(rows, cols // 64)).astype(np.float32)
    s_bits = f32_to_bf16(scale)
    bias = -8.0 * bf16_to_f32(s_bits) + rng.normal(0.0, 1e-3, size=scale.shape).astype(np.float32)
    return packed, s_bits, f32_to_bf16(bias.astype(np.float32))


def bf16_normal(rng: np.random.Generator, shape, std: float = 1.0) -> np.ndarray:
    return f32_to_bf16(rng.normal(0.0, std, size=shape).astype(np.float32))


def unpack_q4(packed: np.ndarray) -> np.ndarray:
    """u32 [rows][words] -> uint8 nibbles [rows][words*8], low nibble first."""
    p = np.asarray(packed, dtype=np.uint32)
    shifts = (4 * np.arange(8, dtype=np.uint32))
    return ((p[..., None] >> shifts) & 0xF).astype(np.uint8).reshape(p.shape[0], -1)


def pack_q4(q: np.ndarray) -> np.ndarray:
    """uint8 nibbles [rows][cols] -> u32 [rows][cols/8] (pack_q4, metal_runtime.rs:11962)."""
    q = np.asarray(q, dtype=np.uint32).reshape(q.shape[0], -1, 8)
    shifts = (4 * np.arange(8, dtype=np.uint32))
    return np.bitwise_or.reduce(q << shifts, axis=-1).astype(np.uint32)
