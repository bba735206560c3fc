"""Depthwise causal 1-D convolution on MI355X — drop-in for the reference's
kernels/causal_conv1d/kernel.py (``custom_kernel((x, weight, bias))``, :170-230).

The work is done by ``thm_causal_conv1d_fwd`` in libtheorem_mi355x.so (a
gfx950 HIP kernel streaming x once with 16-byte vectors); this module only
checks the contract and allocates the output, as the reference launcher does.

Differences from the reference launcher, all extensions:
  * bf16 x/weight/bias are accepted (the reference asserts fp32, :187);
  * ``activation="silu"`` fuses x*sigmoid(x) (the reference has none);
  * ``bias`` may be None.
"""
from __future__ import annotations

import torch

from .. import _capi

__all__ = ["custom_kernel"]

_ACT = {None: _capi.THM_ACT_NONE, "none": _capi.THM_ACT_NONE, "silu": _capi.THM_ACT_SILU}


def custom_kernel(data: tuple, activation: str | None = None) -> torch.Tensor:
    """Run the causal conv.

    Args:
        data: (x, weight, bias) with x [B, D, S], weight [D, W], bias [D] (or None),
            contiguous, on the GPU; x float32 or bfloat16, weight/bias float32 or
            bfloat16.
        activation: None (reference behaviour) or "silu".

    Returns:
        out [B, D, S], dtype of x (``torch.empty_like(x)``, as the reference).
    """
    x, weight, bias = data
    assert x.is_contiguous(), "x must be contiguous (B, D, S)"
    assert weight.is_contiguous(), "weight must be contiguous (D, W)"
    assert bias is None or bias.is_contiguous(), "bias must be contiguous (D,)"
    B, D, S = x.shape
    Dw, W = weight.shape
    assert D == Dw, f"channel mismatch: x has D={D}, weight has D={Dw}"
    if bias is not None:
        assert bias.shape == (D,), f"bias shape {tuple(bias.shape)} != ({D},)"
        assert bias.dtype == weight.dtype, "bias and weight must share a dtype"
    if activation not in _ACT:
        raise ValueError(f"activation must be None or 'silu', got {activation!r}")
    _capi.require_device(x, weight, bias)
    xd = _capi.dtype_code(x, "x")
    wd = _capi.dtype_code(weight, "weight")

    out = torch.empty_like(x)
    lib = _capi.load_library()
    status = lib.thm_causal_conv1d_fwd(
        _capi.ptr(x), _capi.ptr(weight), _capi.ptr(bias), _capi.ptr(out),
        B, D, S, W, xd, wd, _ACT[activation], _capi.stream_of(x),
    )
    _capi.check(status, "thm_causal_conv1d_fwd")
    return out
