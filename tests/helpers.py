"""Small helpers shared by the tests."""
from __future__ import annotations

import numpy as np
import torch


def assert_close(received, expected, rtol: float, atol: float, what: str = "") -> None:
    """|r - e| <= atol + rtol |e| elementwise (the reference's verbose_allclose rule,
    utils.py:71-74), NaN/Inf patterns must match; arrays or tensors, compared in float64."""
    r = received.detach().double().cpu().numpy() if isinstance(received, torch.Tensor) else np.asarray(received, dtype=np.float64)
    e = expected.detach().double().cpu().numpy() if isinstance(expected, torch.Tensor) else np.asarray(expected, dtype=np.float64)
    assert r.shape == e.shape, f"{what}: shape {r.shape} != {e.shape}"
    assert np.array_equal(np.isnan(r), np.isnan(e)), f"{what}: NaN pattern mismatch"
    assert np.array_equal(np.isinf(r), np.isinf(e)), f"{what}: Inf pattern mismatch"
    fin = np.isfinite(r) & np.isfinite(e)
    diff = np.where(fin, np.abs(r - e), 0.0)
    tol = atol + rtol * np.abs(e)
    bad = fin & (diff > tol)
    if bad.any():
        idx = np.argwhere(bad)[:5]
        detail = "; ".join(f"{tuple(i)}: got {r[tuple(i)]:.6g} want {e[tuple(i)]:.6g}" for i in idx)
        raise AssertionError(f"{what}: {int(bad.sum())} elements exceed tol (rtol={rtol}, atol={atol}); "
                             f"max|diff|={diff.max():.3e}; {detail}")


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float values to the nearest bf16 (RNE) and return them as float64."""
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).double().numpy()
