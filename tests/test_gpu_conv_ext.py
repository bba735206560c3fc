"""GPU parity of the causal-conv extensions against the CPU oracle: the
channels-last layout ([B, S, D] storage, thm_causal_conv1d_fwd_channels_last)
and the decode step with a rolling state (thm_causal_conv1d_update).

Tolerances: 1e-4 for fp32 inputs (the reference's conv tolerance), 1e-2 for
bf16 (outputs rounded to bf16)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import conv as oconv
from tests.helpers import assert_close
from theorem_amd.kernels import causal_conv1d

pytestmark = pytest.mark.gpu


def _inputs(B, D, S, W, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, D, S, generator=g)
    w = torch.randn(D, W, generator=g) / 2
    b = torch.randn(D, generator=g) * 0.1
    return x.to(dtype), w.to(dtype), b.to(dtype)


def _cl_view(x, dev):
    """x [B, D, S] -> the same values as a channels-last view (storage [B, S, D])."""
    return x.transpose(1, 2).contiguous().to(dev).transpose(1, 2)


def _oracle(x, w, b, act=None):
    e = oconv.causal_conv1d_numpy(x.double().numpy(), w.double().numpy(),
                                  None if b is None else b.double().numpy(), dtype=np.float64)
    return oconv.silu(e) if act == "silu" else e


@pytest.mark.parametrize("W", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("D,S", [(512, 200), (96, 64), (130, 33)])
def test_channels_last_matches_oracle(dev, W, dtype, D, S):
    x, w, b = _inputs(2, D, S, W, dtype, seed=W + D)
    xv = _cl_view(x, dev)
    assert not xv.is_contiguous() and xv.stride(1) == 1
    out = causal_conv1d.custom_kernel((xv, w.to(dev), b.to(dev)))
    torch.cuda.synchronize()
    assert out.stride() == xv.stride() and out.dtype == dtype
    tol = 1e-4 if dtype == torch.float32 else 1e-2
    assert_close(out, _oracle(x, w, b), tol, tol, f"channels-last W={W} D={D} S={S} {dtype}")


def test_channels_last_silu_no_bias_and_equals_contiguous(dev):
    x, w, b = _inputs(3, 256, 300, 4, torch.float32, seed=1)
    xv = _cl_view(x, dev)
    out = causal_conv1d.custom_kernel((xv, w.to(dev), None), activation="silu")
    ref = causal_conv1d.custom_kernel((x.to(dev), w.to(dev), None), activation="silu")
    torch.cuda.synchronize()
    assert_close(out, _oracle(x, w, None, "silu"), 1e-4, 1e-4, "silu")
    # Both layouts run the same arithmetic order: identical bits.
    assert torch.equal(out.contiguous(), ref)


@pytest.mark.parametrize("W,Ls", [(4, 3), (4, 8), (1, 0), (2, 1)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_update_decode_equals_full_conv(dev, W, Ls, dtype):
    # Token-by-token decode from a zero state reproduces the full-sequence
    # kernel, and the final state is the last Ls inputs.
    B, D, S = 2, 48, 24
    x, w, b = _inputs(B, D, S, W, dtype, seed=W * 10 + Ls)
    xd, wd, bd = x.to(dev), w.to(dev), b.to(dev)
    state = torch.zeros(B, D, Ls, dtype=dtype, device=dev)
    outs = [causal_conv1d.causal_conv1d_update(xd[:, :, t], state, wd, bd) for t in range(S)]
    full = causal_conv1d.custom_kernel((xd.contiguous(), wd, bd))
    torch.cuda.synchronize()
    dec = torch.stack(outs, dim=-1)
    assert dec.dtype == dtype
    assert torch.equal(dec, full), "decode differs from the full-sequence conv"
    if Ls:
        assert torch.equal(state, xd[:, :, S - Ls:])


@pytest.mark.parametrize("act", [None, "silu"])
def test_update_chunked_vs_oracle(dev, act):
    # A multi-sample step (L = 5) from a random state, against the oracle.
    B, D, L, W, Ls = 3, 40, 5, 4, 6
    g = torch.Generator().manual_seed(3)
    x = torch.randn(B, D, L, generator=g)
    st = torch.randn(B, D, Ls, generator=g)
    w = torch.randn(D, W, generator=g)
    b = torch.randn(D, generator=g)
    state = st.to(dev)
    out = causal_conv1d.causal_conv1d_update(x.to(dev), state, w.to(dev), b.to(dev), activation=act)
    torch.cuda.synchronize()
    e, est = oconv.causal_conv1d_update_ref(x.double().numpy(), st.double().numpy(), w.double().numpy(),
                                            b.double().numpy())
    if act == "silu":
        e = oconv.silu(e)
    assert_close(out, e, 1e-5, 1e-5, f"update act={act}")
    assert_close(state, est, 0, 0, "new state")


def test_update_rejects_short_state(dev):
    x = torch.zeros(1, 4, 1, device=dev)
    with pytest.raises(ValueError):
        causal_conv1d.causal_conv1d_update(x, torch.zeros(1, 4, 2, device=dev), torch.zeros(4, 4, device=dev))
