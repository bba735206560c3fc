"""Pins the causal-conv oracle (C and NumPy restatements of
scripts/cpu_reference.py:40-63) against the mathematics and a library routine."""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import conv


def _inputs(B, D, S, W, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((B, D, S), dtype=np.float32),
            rng.standard_normal((D, W), dtype=np.float32),
            rng.standard_normal((D,), dtype=np.float32))


SHAPES = [(1, 64, 64, 4), (2, 128, 128, 4), (1, 256, 256, 3), (1, 128, 64, 8), (4, 64, 128, 4),
          (1, 3, 17, 1), (2, 5, 9, 7)]


@pytest.mark.parametrize("B,D,S,W", SHAPES)
def test_c_numpy_torch_agree(B, D, S, W):
    x, w, b = _inputs(B, D, S, W, 1)
    out_c = conv.causal_conv1d_c(x, w, b)
    out_np = conv.causal_conv1d_numpy(x, w, b)
    # Same operation order (bias, then taps in order, mul-then-add in fp32): bit-identical.
    assert np.array_equal(out_c, out_np)
    # Library routine: torch CPU depthwise conv1d (cpu_reference.py:66-83 check, atol 1e-4).
    ref = F.conv1d(F.pad(torch.from_numpy(x), (W - 1, 0)), torch.from_numpy(w).unsqueeze(1),
                   bias=torch.from_numpy(b), groups=D).numpy()
    assert np.abs(out_c - ref).max() <= 1e-4


@pytest.mark.parametrize("B,D,S,W", [(1, 3, 11, 4), (2, 2, 9, 8), (1, 4, 5, 3)])
def test_bruteforce(B, D, S, W):
    x, w, b = _inputs(B, D, S, W, 2)
    assert np.abs(conv.causal_conv1d_c(x, w, b) - conv.causal_conv1d_bruteforce(x, w, b)).max() < 1e-5


@pytest.mark.parametrize("W", [1, 2, 3, 4, 8])
def test_impulse_pins_tap_order(W):
    # x = delta at t0  ->  out[t0 + j] = b + w[W-1-j] for 0 <= j < W, = b elsewhere.
    D, S, t0 = 3, 32, 10
    x = np.zeros((1, D, S), dtype=np.float32)
    x[0, :, t0] = 1.0
    w = np.arange(1, D * W + 1, dtype=np.float32).reshape(D, W)
    b = np.array([0.5, -1.0, 2.0], dtype=np.float32)
    out = conv.causal_conv1d_c(x, w, b)
    for d in range(D):
        exp = np.full(S, b[d], dtype=np.float32)
        for j in range(W):
            exp[t0 + j] = b[d] + w[d, W - 1 - j]
        assert np.array_equal(out[0, d], exp)


def test_width1_closed_form():
    x, w, b = _inputs(2, 8, 33, 1, 3)
    assert np.array_equal(conv.causal_conv1d_c(x, w, b), w[None, :, 0:1] * x + b[None, :, None])


def test_causality_and_linearity():
    x, w, b = _inputs(1, 4, 40, 4, 4)
    base = conv.causal_conv1d_numpy(x, w, b, dtype=np.float64)
    x2 = x.copy()
    x2[..., 25:] += 7.0                          # future perturbation
    pert = conv.causal_conv1d_numpy(x2, w, b, dtype=np.float64)
    assert np.array_equal(base[..., :25], pert[..., :25])
    y = np.random.default_rng(5).standard_normal(x.shape).astype(np.float32)
    lhs = conv.causal_conv1d_numpy(2 * x.astype(np.float64) + y, w, None, dtype=np.float64)
    rhs = 2 * conv.causal_conv1d_numpy(x, w, None, dtype=np.float64) + conv.causal_conv1d_numpy(y, w, None, dtype=np.float64)
    assert np.abs(lhs - rhs).max() < 1e-9


def test_mutation_is_caught():
    # A plausible mistake (reversed taps) must fail the impulse check above.
    x = np.zeros((1, 1, 16), dtype=np.float32)
    x[0, 0, 4] = 1.0
    w = np.array([[1.0, 2.0, 3.0]], dtype=np.float32)
    good = conv.causal_conv1d_c(x, w, None)
    bad = conv.causal_conv1d_c(x, w[:, ::-1].copy(), None)
    assert good[0, 0, 4] == 3.0 and not np.array_equal(good, bad)


def test_silu_pins():
    # silu(x) = x * sigmoid(x): torch's library routine, the fixed point
    # silu(0) = 0, the limits x (x -> +inf) and 0 (x -> -inf), and
    # silu(x) - silu(-x) = x (an odd-part identity a sign slip breaks).
    x = np.linspace(-30, 30, 2001)
    got = conv.silu(x)
    np.testing.assert_allclose(got, F.silu(torch.from_numpy(x)).numpy(), rtol=1e-12, atol=1e-12)
    assert conv.silu(np.array([0.0]))[0] == 0.0
    np.testing.assert_allclose(conv.silu(np.array([40.0, -40.0])), [40.0, 0.0], atol=1e-12)
    np.testing.assert_allclose(got - conv.silu(-x), x, atol=1e-12)


def test_update_ref_pins():
    # Token-by-token decode from a zero state reproduces the full-sequence conv
    # (the NumPy restatement), the state is the last L_s samples, and a chunked
    # decode (L > 1) equals the token-by-token one.
    rng = np.random.default_rng(5)
    for W, Ls in ((4, 3), (4, 6), (1, 0), (3, 2)):
        x = rng.standard_normal((2, 3, 20))
        w = rng.standard_normal((3, W))
        b = rng.standard_normal(3)
        full = conv.causal_conv1d_numpy(x, w, b, dtype=np.float64)
        st = np.zeros((2, 3, Ls))
        outs = []
        for t in range(20):
            o, st = conv.causal_conv1d_update_ref(x[:, :, t:t + 1], st, w, b)
            outs.append(o)
        np.testing.assert_allclose(np.concatenate(outs, axis=2), full, rtol=1e-12, atol=1e-12)
        if Ls:
            np.testing.assert_array_equal(st, x[:, :, 20 - Ls:])
        st2 = np.zeros((2, 3, Ls))
        o1, st2 = conv.causal_conv1d_update_ref(x[:, :, :7], st2, w, b)
        o2, st2 = conv.causal_conv1d_update_ref(x[:, :, 7:], st2, w, b)
        np.testing.assert_allclose(np.concatenate([o1, o2], axis=2), full, rtol=1e-12, atol=1e-12)
        np.testing.assert_array_equal(st2, st)
