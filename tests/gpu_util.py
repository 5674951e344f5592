"""Helpers for GPU parity tests: numpy <-> device tensors and tolerances."""
from __future__ import annotations

import numpy as np


def to_dev(a: np.ndarray, dev):
    import torch
    a = np.ascontiguousarray(a)
    view = {np.dtype(np.uint16): np.int16, np.dtype(np.uint32): np.int32}.get(a.dtype)
    if view is not None:
        a = a.view(view)
    return torch.from_numpy(a).to(dev)


def from_dev(t, dtype=None) -> np.ndarray:
    import torch
    torch.cuda.synchronize()
    a = t.detach().cpu().numpy()
    if dtype is not None:
        a = a.view(dtype)
    return a


def empty_bf16(shape, dev):
    import torch
    return torch.full(shape, -1, dtype=torch.int16, device=dev)  # NaN-ish fill to catch unwritten cells


def bf16_dev_to_f32(t) -> np.ndarray:
    b = from_dev(t, np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def assert_bf16_close(got_f32: np.ndarray, ref_f32: np.ndarray, rel: float = 2e-3, what: str = ""):
    """bf16 outputs: max |got - ref| <= rel * max |ref| (normwise, ref in fp32/fp64)."""
    got = np.asarray(got_f32, np.float64)
    ref = np.asarray(ref_f32, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    scale = max(np.max(np.abs(ref)), 1e-30)
    err = np.max(np.abs(got - ref)) / scale
    assert err <= rel, f"{what}: max rel err {err:.3e} > {rel:.1e}"
    return err
