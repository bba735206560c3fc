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
        if key in data and data[key] != val:
            raise AssertionError(f"data[{key!r}]={data[key]} disagrees with the tensors ({val})")
    fp = _capi.fastpath()
    if fp is not None:
        r = _capi.fast_result(fp.h(k, w, vu, g, h0, delta, want_vn, want_ht), "thm_chunk_fwd_h")
        if r is not None:
            if delta:
                return r
            return (r[0], r[2]) if want_ht else r[0]
    assert T % CHUNK_SIZE == 0, f"T={T} must be divisible by {CHUNK_SIZE}"
    NT = T // CHUNK_SIZE
    if vu.shape[:3] != (B, T, H) or (w is not None and w.shape != k.shape) or (
            g is not None and g.shape != (B, T, H)) or (h0 is not None and h0.shape != (B, H, K, V)):
        raise AssertionError(f"shapes: k {tuple(k.shape)}, v/u {tuple(vu.shape)}, "
                             f"w {None if w is None else tuple(w.shape)}, g {None if g is None else tuple(g.shape)}, "
                             f"initial_state {None if h0 is None else tuple(h0.shape)}")
    if k.dtype is not vu.dtype or (w is not None and w.dtype is not k.dtype):
        raise AssertionError("k, v/u, w must share a dtype")
    f32 = torch.float32
    if (g is not None and g.dtype is not f32) or (h0 is not None and h0.dtype is not f32):
        raise AssertionError("g and initial_state must be float32")
    code = _capi.dtype_code(k, "k")
    (pk, pw, pu, pg, ph0), keep = _capi.dev_ptrs(k, w, vu, g, h0)

    dev = _capi.device_of(k)
    h = torch.empty((B, NT, H, K, V), dtype=f32, device=dev)
    v_new = (torch.empty_like(vu) if vu.is_contiguous() else vu.new_empty(vu.shape)) if want_vn else None
    ht = torch.empty((B, H, K, V), dtype=f32, device=dev) if want_ht else None
    status = _capi.load_library().thm_chunk_fwd_h(
        pk, pw, pu, pg, ph0, h.data_ptr(), None if v_new is None else v_new.data_ptr(),
        None if ht is None else ht.data_ptr(),
        B, T, H, K, V, CHUNK_SIZE, code, _capi.THM_H_DELTA if delta else 0, _capi.stream_of(k))
    _capi.check(status, "thm_chunk_fwd_h")
    if delta:
        return h, v_new, ht
    return (h, ht) if want_ht else h
