"""Gated DeltaNet inter-chunk state recurrence on MI355X — drop-in for the
reference's kernels/chunk_fwd_h/kernel.py (``custom_kernel(dict) -> h``, :141-191).

The work is done by ``thm_chunk_fwd_h`` in libtheorem_mi355x.so.

Reference form (the reference's contract): ``data`` has k, v, g (+ B, T, H,
K, V); returns h [B, T/64, H, K, V] fp32 holding the state after each chunk.

Delta-rule form (extension, selected by the keys ``w`` and ``u``): returns
``(h, v_new, final_state)`` with h[c] the state BEFORE chunk c,
v_new = u - w.S (dtype of u, or None when ``save_new_value`` is False) and the
final state (fp32, or None unless ``output_final_state``).  Optional
``initial_state`` [B, H, K, V] fp32 seeds the recurrence in either form; in
the reference form ``output_final_state`` makes the result ``(h, final_state)``.
k / v / w / u may be bf16; g, the states and h are fp32.
"""
from __future__ import annotations

import torch

from .. import _capi

__all__ = ["custom_kernel"]

CHUNK_SIZE = 64


def custom_kernel(data):
    k = data["k"]
    delta = "w" in data or "u" in data
    vu = data["u"] if delta else data["v"]
    w = data["w"] if delta else None
    g = data.get("g")
    h0 = data.get("initial_state")
    want_ht = bool(data.get("output_final_state", False))
    want_vn = delta and bool(data.get("save_new_value", True))
    B, T, H, K = k.shape
    V = vu.shape[-1]
    for key, val in (("B", B), ("T", T), ("H", H), ("K", K), ("V", V)):
        assert data.get(key, val) == val, f"data[{key!r}]={data[key]} disagrees with the tensors ({val})"
    assert T % CHUNK_SIZE == 0, f"T={T} must be divisible by {CHUNK_SIZE}"
    NT = T // CHUNK_SIZE
    assert vu.shape[:3] == (B, T, H)
    assert w is None or w.shape == (B, T, H, K)
    assert g is None or g.shape == (B, T, H)
    assert h0 is None or h0.shape == (B, H, K, V)
    assert k.dtype == vu.dtype and (w is None or w.dtype == k.dtype), "k, v/u, w must share a dtype"
    _capi.require_device(k, w, vu, g, h0)
    _capi.require_f32(g, "g")
    _capi.require_f32(h0, "initial_state")
    code = _capi.dtype_code(k, "k")
    k, w, vu, g, h0 = (_capi.prep(t, "") for t in (k, w, vu, g, h0))

    h = torch.empty(B, NT, H, K, V, device=k.device, dtype=torch.float32)
    v_new = torch.empty_like(vu) if want_vn else None
    ht = torch.empty(B, H, K, V, device=k.device, dtype=torch.float32) if want_ht else None
    status = _capi.load_library().thm_chunk_fwd_h(
        _capi.ptr(k), _capi.ptr(w), _capi.ptr(vu), _capi.ptr(g), _capi.ptr(h0),
        _capi.ptr(h), _capi.ptr(v_new), _capi.ptr(ht),
        B, T, H, K, V, CHUNK_SIZE, code, _capi.THM_H_DELTA if delta else 0, _capi.stream_of(k))
    _capi.check(status, "thm_chunk_fwd_h")
    if delta:
        return h, v_new, ht
    return (h, ht) if want_ht else h
