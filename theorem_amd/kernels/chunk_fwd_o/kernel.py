"""Gated DeltaNet chunkwise output on MI355X — drop-in for the reference's
kernels/chunk_fwd_o/kernel.py (``custom_kernel(dict) -> o``, :146-212).

The work is done by ``thm_chunk_fwd_o`` in libtheorem_mi355x.so; this module
checks the contract (NT == T / 64, kernel.py:178-179) and allocates o with q's
dtype (kernel.py:183).  Extensions: bf16 q / k / v (o then bf16); g may be None.
"""
from __future__ import annotations

from typing import Any, Dict

import torch

from .. import _capi

__all__ = ["custom_kernel"]

BT = 64


def custom_kernel(data: Dict[str, Any]) -> torch.Tensor:
    """o = scale (mask_incl(q k^T e^{g_i - g_j}) v + e^{g} q h[c]); o [B, T, H, V]."""
    q, k, v, g, h = data["q"], data["k"], data["v"], data.get("g"), data["h"]
    scale = float(data["scale"])
    B, T, H, K = q.shape
    V = v.shape[-1]
    NT = h.shape[1]
    assert T % BT == 0, f"T={T} must be divisible by BT={BT}"
    assert NT == T // BT, f"NT={NT} must equal T/BT={T // BT}"
    assert k.shape == (B, T, H, K) and v.shape[:3] == (B, T, H) and h.shape == (B, NT, H, K, V)
    assert g is None or g.shape == (B, T, H)
    assert q.dtype == k.dtype == v.dtype, "q, k, v must share a dtype"
    _capi.require_device(q, k, v, g, h)
    _capi.require_f32(g, "g")
    _capi.require_f32(h, "h")
    code = _capi.dtype_code(q, "q")
    q, k, v, g, h = (_capi.prep(t, "") for t in (q, k, v, g, h))
    o = torch.empty(B, T, H, V, dtype=q.dtype, device=q.device)
    status = _capi.load_library().thm_chunk_fwd_o(
        _capi.ptr(q), _capi.ptr(k), _capi.ptr(v), _capi.ptr(g), _capi.ptr(h), _capi.ptr(o), scale,
        B, T, H, K, V, BT, code, _capi.stream_of(q))
    _capi.check(status, "thm_chunk_fwd_o")
    return o
