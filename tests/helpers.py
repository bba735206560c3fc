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


# --------------------------------------------------------------------------- planted carry mistakes
# Copies of the delta-form state recurrence (oracle/deltanet.py
# chunk_fwd_h_delta, float64) with one plausible mistake in the inter-chunk
# carry.  A parity test feeds them the inputs it gives the GPU and checks that
# each mistake moves the result beyond the tolerance, so that matching the
# exact oracle within that tolerance shows the carry was computed right.

def h_delta_carry_mutant(k, w, u, g, h0, mode: str, bt: int = 64):
    """(h [B, NT, H, K, V] before each chunk, v_new [B, T, H, V], final S) of
    the delta form with the carried state treated per ``mode``:
      "dropped"      S <- (k e^{g_last - g})^T v_new          (no e^{g_last} S term)
      "double_decay" S <- e^{2 g_last} S + (k e^{g_last - g})^T v_new
    ``w`` None means w = 0 (the reference form, stored one chunk later)."""
    B, T, H, K = k.shape
    V = u.shape[-1]
    NT = T // bt

    def ch(x):
        return np.moveaxis(np.asarray(x, dtype=np.float64).reshape(B, NT, bt, H, *x.shape[3:]), 3, 1)

    kc, uc = ch(k), ch(u)
    wc = ch(w) if w is not None else np.zeros_like(kc)
    gc = ch(g) if g is not None else np.zeros(kc.shape[:4])
    S = np.zeros((B, H, K, V)) if h0 is None else np.asarray(h0, dtype=np.float64).copy()
    h = np.zeros((B, NT, H, K, V))
    vn = np.zeros_like(uc)
    for c in range(NT):
        h[:, c] = S
        vn[:, :, c] = uc[:, :, c] - wc[:, :, c] @ S
        gl = gc[:, :, c, -1]
        kg = kc[:, :, c] * np.exp(gl[..., None] - gc[:, :, c])[..., None]
        upd = np.swapaxes(kg, -1, -2) @ vn[:, :, c]
        if mode == "dropped":
            S = upd
        elif mode == "double_decay":
            S = S * np.exp(2 * gl)[..., None, None] + upd
        else:
            raise ValueError(mode)
    return h, np.moveaxis(vn, 1, 3).reshape(B, T, H, V), S


def tokens_chunk_reset(q, k, v, beta, a, scale: float, bt: int = 64):
    """The token-level gated delta rule with the state reset to zero at every
    chunk boundary (the inter-chunk carry dropped); o [B, T, H, V]."""
    from oracle import deltanet as odn
    T = k.shape[1]
    outs = [odn.gated_delta_rule_tokens(q[:, t:t + bt], k[:, t:t + bt], v[:, t:t + bt], beta[:, t:t + bt],
                                        a[:, t:t + bt], scale)[0] for t in range(0, T, bt)]
    return np.concatenate(outs, axis=1)


def assert_differs(mutant, expected, rtol: float, atol: float, what: str, min_frac: float = 1e-3) -> float:
    """At least ``min_frac`` of the elements of ``mutant`` lie outside the
    tolerance band around ``expected`` (so a result equal to the mutant would
    fail assert_close); returns that fraction."""
    m = np.asarray(mutant, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    frac = float((np.abs(m - e) > atol + rtol * np.abs(e)).mean())
    assert frac >= min_frac, f"{what}: the planted mistake stays within tolerance ({frac:.2e} of elements outside)"
    return frac
