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
    fp = _capi.fastpath()
    if fp is not None:
        o = _capi.fast_result(fp.o(q, k, v, g, h, scale), "thm_chunk_fwd_o")
        if o is not None:
            return o
    B, T, H, K = q.shape
    V = v.shape[-1]
    NT = h.shape[1]
    assert T % BT == 0, f"T={T} must be divisible by BT={BT}"
    assert NT == T // BT, f"NT={NT} must equal T/BT={T // BT}"
    if k.shape != q.shape or v.shape[:3] != (B, T, H) or h.shape != (B, NT, H, K, V) or (
            g is not None and g.shape != (B, T, H)):
        raise AssertionError(f"shapes: q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}, "
                             f"h {tuple(h.shape)}, g {None if g is None else tuple(g.shape)}")
    if not (q.dtype is k.dtype is v.dtype):
        raise AssertionError("q, k, v must share a dtype")
    if h.dtype is not torch.float32 or (g is not None and g.dtype is not torch.float32):
        raise AssertionError("g and h must be float32")
    code = _capi.dtype_code(q, "q")
    (pq, pk, pv, pg, ph), keep = _capi.dev_ptrs(q, k, v, g, h)
    # o has q's dtype (kernel.py:183), which v shares, and v's shape.
    o = torch.empty_like(v) if v.is_contiguous() else v.new_empty(v.shape)
    status = _capi.load_library().thm_chunk_fwd_o(
        pq, pk, pv, pg, ph, o.data_ptr(), scale, B, T, H, K, V, BT, code, _capi.stream_of(q))
    _capi.check(status, "thm_chunk_fwd_o")
    return o
