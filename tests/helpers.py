"""Shared helpers of the parity tests (host side: numpy <-> torch device buffers,
the fp16 tolerance of the path)."""
from __future__ import annotations

import numpy as np


def dev(a: np.ndarray):
    """numpy -> device tensor with the same bytes (uint32 travels as int32)."""
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a).cuda()


def host(t, dtype=None) -> np.ndarray:
    import torch
    torch.cuda.synchronize()
    a = t.cpu().numpy()
    if dtype is not None:
        a = a.view(dtype)
    return a


def empty(shape, dtype):
    import torch
    return torch.empty(shape, dtype=dtype, device="cuda")


def ulp16(x: np.ndarray) -> np.ndarray:
    """Spacing of fp16 values at |x| (subnormal spacing 2^-24 near zero)."""
    ax = np.abs(np.asarray(x, np.float64))
    e = np.floor(np.log2(np.maximum(ax, 2.0 ** -14)))
    return 2.0 ** (e - 10)


def assert_fp16_close(got16: np.ndarray, exact: np.ndarray, bound: np.ndarray, ref16: np.ndarray | None = None,
                      min_identical: float = 0.95, what: str = "", max_floor_frac: float = 0.01):
    """Tolerance of the fp16 outputs: within 2 fp16 ulp or 1e-3 relative of the
    exact (double) oracle value, plus the fp32-accumulation floor
    2^-20 * sum|terms| that matters only for outputs near zero (cancellation:
    an fp32 sum of K terms carries an error of order 2^-24 * sum|terms|, which
    2 ulp of a near-zero result cannot hold).  At most max_floor_frac of the
    outputs may need the floor.  Also requires that most outputs round to the
    same fp16 as the oracle."""
    g = got16.astype(np.float64).reshape(-1)
    ex = np.asarray(exact, np.float64).reshape(-1)
    bd = np.asarray(bound, np.float64).reshape(-1)
    assert np.all(np.isfinite(g)), f"{what}: non-finite outputs"
    err = np.abs(g - ex)
    tol = np.maximum(2 * ulp16(ex), 1e-3 * np.abs(ex)) + 2.0 ** -20 * bd
    need_floor = np.mean(err > np.maximum(2 * ulp16(ex), 1e-3 * np.abs(ex)))
    assert need_floor <= max_floor_frac, f"{what}: {need_floor:.4f} of outputs need the fp32-accumulation floor"
    bad = np.nonzero(err > tol)[0]
    assert bad.size == 0, (f"{what}: {bad.size} outputs out of tolerance, first at {bad[0]}: "
                           f"got {g[bad[0]]!r} exact {ex[bad[0]]!r} tol {tol[bad[0]]!r}")
    if ref16 is not None:
        same = np.mean(got16.reshape(-1).view(np.uint16) == ref16.reshape(-1).view(np.uint16))
        assert same >= min_identical, f"{what}: only {same:.3f} of outputs bit-identical to the oracle"
