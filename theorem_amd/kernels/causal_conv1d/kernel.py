"""Depthwise causal 1-D convolution on MI355X — drop-in for the reference's
kernels/causal_conv1d/kernel.py (``custom_kernel((x, weight, bias))``, :170-230).

The work is done by ``thm_causal_conv1d_fwd`` in libtheorem_mi355x.so (a
gfx950 HIP kernel streaming x once with 16-byte vectors); this module only
checks the contract and allocates the output, as the reference launcher does.

Differences from the reference launcher, all extensions:
  * bf16 x/weight/bias are accepted (the reference asserts fp32, :187);
  * ``activation="silu"`` fuses x*sigmoid(x) (the reference has none);
  * ``bias`` may be None;
  * x may also be channels-last: a [B, D, S] view of a contiguous [B, S, D]
    tensor (stride(1) == 1), run by ``thm_causal_conv1d_fwd_channels_last``;
    the output then has the same layout (``torch.empty_like`` keeps strides).
``causal_conv1d_update`` is the decode step with a rolling state (no
counterpart in the reference).
"""
from __future__ import annotations

import torch

from .. import _capi

__all__ = ["custom_kernel", "causal_conv1d_update"]

_ACT = {None: _capi.THM_ACT_NONE, "none": _capi.THM_ACT_NONE, "silu": _capi.THM_ACT_SILU}


def _check_params(weight, bias, D, activation):
    assert weight.is_contiguous(), "weight must be contiguous (D, W)"
    assert bias is None or bias.is_contiguous(), "bias must be contiguous (D,)"
    Dw, W = weight.shape
    assert D == Dw, f"channel mismatch: x has D={D}, weight has D={Dw}"
    if bias is not None:
        assert bias.shape == (D,), f"bias shape {tuple(bias.shape)} != ({D},)"
        assert bias.dtype == weight.dtype, "bias and weight must share a dtype"
    if activation not in _ACT:
        raise ValueError(f"activation must be None or 'silu', got {activation!r}")
    return W


def _is_channels_last(x: torch.Tensor) -> bool:
    B, D, S = x.shape
    return x.stride(1) == 1 and x.stride(2) == D and x.stride(0) == D * S and D > 1


def custom_kernel(data: tuple, activation: str | None = None) -> torch.Tensor:
    """Run the causal conv.

    Args:
        data: (x, weight, bias) with x [B, D, S] (contiguous, or a channels-last
            view of [B, S, D]), weight [D, W], bias [D] (or None), on the GPU;
            x float32 or bfloat16, weight/bias float32 or bfloat16.
        activation: None (reference behaviour) or "silu".

    Returns:
        out [B, D, S], dtype and layout of x (``torch.empty_like(x)``).
    """
    x, weight, bias = data
    act = _ACT.get(activation)
    fp = _capi.fastpath() if act is not None else None
    if fp is not None:
        out = _capi.fast_result(fp.conv1d(x, weight, bias, act), "thm_causal_conv1d_fwd")
        if out is not None:
            return out
    B, D, S = x.shape
    channels_last = not x.is_contiguous() and _is_channels_last(x)
    assert x.is_contiguous() or channels_last, "x must be contiguous (B, D, S) or channels-last"
    W = _check_params(weight, bias, D, activation)
    _capi.require_device(x, weight, bias)
    xd = _capi.dtype_code(x, "x")
    wd = _capi.dtype_code(weight, "weight")

    out = torch.empty_like(x)
    lib = _capi.load_library()
    if channels_last:
        status = lib.thm_causal_conv1d_fwd_channels_last(
            _capi.ptr(x), _capi.ptr(weight), _capi.ptr(bias), _capi.ptr(out),
            B, S, D, W, xd, wd, _ACT[activation], _capi.stream_of(x))
        _capi.check(status, "thm_causal_conv1d_fwd_channels_last")
    else:
        status = lib.thm_causal_conv1d_fwd(
            _capi.ptr(x), _capi.ptr(weight), _capi.ptr(bias), _capi.ptr(out),
            B, D, S, W, xd, wd, _ACT[activation], _capi.stream_of(x))
        _capi.check(status, "thm_causal_conv1d_fwd")
    return out


def causal_conv1d_update(x: torch.Tensor, conv_state: torch.Tensor, weight: torch.Tensor,
                         bias: torch.Tensor | None = None, activation: str | None = None) -> torch.Tensor:
    """Decode step: x [B, D] or [B, D, L] new samples, conv_state [B, D, state_len]
    (state_len >= W - 1, dtype of x) updated in place to the last state_len
    samples of conv_state ++ x.  Returns out like x:
        out[..., t] = act(bias + sum_k weight[:, k] * (conv_state ++ x)[..., state_len - W + 1 + t + k])."""
    squeeze = x.dim() == 2
    if squeeze:
        x = x.unsqueeze(-1)
    B, D, L = x.shape
    x = x.contiguous()  # a strided slice (e.g. one timestep of [B, D, S]) is copied
    assert conv_state.is_contiguous() and conv_state.shape[:2] == (B, D), "conv_state must be [B, D, state_len]"
    assert conv_state.dtype == x.dtype, "conv_state must have the dtype of x"
    W = _check_params(weight, bias, D, activation)
    _capi.require_device(x, conv_state, weight, bias)
    xd = _capi.dtype_code(x, "x")
    wd = _capi.dtype_code(weight, "weight")
    out = torch.empty_like(x)
    status = _capi.load_library().thm_causal_conv1d_update(
        _capi.ptr(x), _capi.ptr(conv_state), _capi.ptr(weight), _capi.ptr(bias), _capi.ptr(out),
        B, D, L, conv_state.shape[2], W, xd, wd, _ACT[activation], _capi.stream_of(x))
    _capi.check(status, "thm_causal_conv1d_update")
    return out.squeeze(-1) if squeeze else out
