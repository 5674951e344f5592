"""Helpers for GPU parity tests: numpy <-> device tensors and tolerances."""
from __future__ import annotations

import os
from contextlib import contextmanager

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


def bf16_half_ulp(v: np.ndarray) -> np.ndarray:
    """Half a bf16 ulp at |v| (bf16 keeps 8 significant bits)."""
    a = np.abs(np.asarray(v, np.float64))
    e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    return np.where(a > 0, 2.0 ** (e - 8), 0.0)


def assert_bf16_close(got_f32: np.ndarray, ref_f32: np.ndarray, rel: float = 1e-4, what: str = ""):
    """bf16 outputs vs an fp32/fp64 oracle.

    The kernel's result before its final bf16 store must lie within
    rel * max|ref| of the oracle: |got - ref| - halfulp_bf16(got) <= rel * max|ref|.
    (The store itself rounds to nearest-even, which alone can move a value by
    up to 2^-8 relative, so it is accounted for separately instead of being
    charged to the arithmetic.)  The default 1e-4 is 20x below the 2e-3 bar
    for bf16 outputs; the largest arithmetic error any GPU test measures
    against its oracle is 3.2e-5 (causal prefill attention), except where a
    test compares against a deliberately different chain and says so.
    QM38_TOL_LOG=<file> appends each call's measured errors to <file>.
    Returns the arithmetic error (normwise).
    """
    got = np.asarray(got_f32, np.float64)
    ref = np.asarray(ref_f32, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    scale = max(np.max(np.abs(ref)), 1e-30)
    excess = np.maximum(np.abs(got - ref) - bf16_half_ulp(got) * (1 + 1e-6), 0.0)
    err = np.max(excess) / scale
    raw = np.max(np.abs(got - ref)) / scale
    log = os.environ.get("QM38_TOL_LOG")  # measured errors, for choosing each test's bound
    if log:
        with open(log, "a") as f:
            test = os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0]
            f.write(f"{test}\t{what}\t{err:.3e}\t{raw:.3e}\t{rel:.1e}\n")
    assert err <= rel, f"{what}: arithmetic rel err {err:.3e} > {rel:.1e} (raw incl. bf16 rounding {raw:.3e})"
    assert raw <= rel + 2.0 ** -8, f"{what}: raw rel err {raw:.3e}"
    return err


@contextmanager
def tuned(**env):
    """A fresh runtime on cuda:0 (torch's current stream) whose planner uses
    the given QM38_* overrides: the library reads them once, when a runtime
    is created.  A value of None leaves that variable unset."""
    import torch
    import qm38
    saved = {k: os.environ.get(k) for k in env}
    try:
        for k, v in env.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = str(v)
        r = qm38.Runtime(0)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    r.set_stream(torch.cuda.current_stream())
    try:
        yield r
    finally:
        torch.cuda.synchronize()
        r.close()
