"""Gated DeltaNet WY recompute on MI355X — drop-in for the reference's
kernels/recompute_w_u/kernel.py (``custom_kernel(Data) -> (w, u)``, :246-248).

The work is done by ``thm_recompute_w_u_fwd`` in libtheorem_mi355x.so; this
module checks the contract and allocates w, u with ``torch.empty_like(k / v)``
as the reference launcher does (kernel.py:202-203).  Extensions: bf16 k / v
(w, u then bf16); g may be None.

``build_A`` is the step before: the WY matrix A of ``_build_A``
(reference.py:48-91) on the GPU (``thm_wy_build_A``).
"""
from __future__ import annotations

import torch

from .. import _capi
from .reference import BT, Data

__all__ = ["custom_kernel", "build_A", "SHAPE_CONFIGS", "SHAPE_LIST"]

# Shapes of the reference's task.yml (tests, then benchmarks).
SHAPE_LIST = [
    {"B": 1, "T": 64, "H": 2, "K": 64, "V": 64},
    {"B": 2, "T": 128, "H": 4, "K": 64, "V": 64},
    {"B": 1, "T": 256, "H": 4, "K": 64, "V": 128},
    {"B": 1, "T": 64, "H": 1, "K": 64, "V": 64},
    {"B": 2, "T": 512, "H": 3, "K": 64, "V": 64},
    {"B": 2, "T": 1024, "H": 3, "K": 64, "V": 64},
]

# Launch configuration per shape.  The HIP kernel uses one rule for every
# shape (one 256-thread workgroup per (b, chunk, head) tile), so this table
# only documents it; it is not a tuning knob.
SHAPE_CONFIGS = {
    (s["B"], s["T"], s["H"], s["K"], s["V"]): {"threads": 256, "tiles": s["B"] * s["H"] * (s["T"] // BT)}
    for s in SHAPE_LIST
}


def _launch(k, v, beta, A, g):
    fp = _capi.fastpath()
    if fp is not None:
        r = _capi.fast_result(fp.wu(k, v, beta, A, g), "thm_recompute_w_u_fwd")
        if r is not None:
            return r
    B, T, H, K = k.shape
    V = v.shape[-1]
    bth = (B, T, H)
    if T % BT or v.shape[:3] != bth or beta.shape != bth or A.shape != (B, T, H, BT) or (
            g is not None and g.shape != bth):
        raise AssertionError(f"shapes: k {tuple(k.shape)}, v {tuple(v.shape)}, beta {tuple(beta.shape)}, "
                             f"A {tuple(A.shape)}, g {None if g is None else tuple(g.shape)} (T % {BT} == 0)")
    f32 = torch.float32
    if beta.dtype is not f32 or A.dtype is not f32 or (g is not None and g.dtype is not f32):
        raise AssertionError("beta, A and g must be float32")
    if k.dtype is not v.dtype:
        raise AssertionError("k and v must share a dtype")
    code = _capi.dtype_code(k, "k")
    (pk, pv, pb, pa, pg), keep = _capi.dev_ptrs(k, v, beta, A, g)
    # Dense, with k's / v's dtype and device (torch.empty_like in kernel.py:202-203);
    # empty_like is the cheapest allocation (~1.2 us against ~1.9 for new_empty)
    # and keeps a dense input's layout.
    w = torch.empty_like(k) if k.is_contiguous() else k.new_empty(k.shape)
    u = torch.empty_like(v) if v.is_contiguous() else v.new_empty(v.shape)
    status = _capi.load_library().thm_recompute_w_u_fwd(
        pk, pv, pb, pa, pg, w.data_ptr(), u.data_ptr(), B, T, H, K, V, BT, code, _capi.stream_of(k))
    _capi.check(status, "thm_recompute_w_u_fwd")
    return w, u


def custom_kernel(data: Data) -> tuple[torch.Tensor, torch.Tensor]:
    """(w, u) = recompute_w_u(k, v, beta, A, g); same dtype as k / v."""
    return _launch(data.k, data.v, data.beta, data.A, data.g)


def build_A(k: torch.Tensor, beta: torch.Tensor, g: torch.Tensor | None, sign: int = -1) -> torch.Tensor:
    """A [B, T, H, 64] fp32, per 64-token chunk A_c = (I + sign M)^{-1} with
    M = strict_lower(beta_i (k_i . k_j) e^{g_i - g_j}).  sign = -1 is the
    reference's ``_build_A`` (reference.py:48-91, (I - M)^{-1}); sign = +1 the
    gated delta rule's (I + M)^{-1}.  k fp32 or bf16; beta, g fp32; g may be None."""
    B, T, H, K = k.shape
    assert T % BT == 0, f"T={T} must be a multiple of {BT}"
    assert beta.shape == (B, T, H) and (g is None or g.shape == (B, T, H))
    assert sign in (1, -1), "sign must be +1 or -1"
    _capi.require_device(k, beta, g)
    for name, t in (("beta", beta), ("g", g)):
        _capi.require_f32(t, name)
    code = _capi.dtype_code(k, "k")
    k, beta, g = (_capi.prep(t, n) for t, n in ((k, "k"), (beta, "beta"), (g, "g")))
    A = torch.empty(B, T, H, BT, dtype=torch.float32, device=k.device)
    status = _capi.load_library().thm_wy_build_A(
        _capi.ptr(k), _capi.ptr(beta), _capi.ptr(g), _capi.ptr(A), B, T, H, K, BT, code, sign,
        _capi.stream_of(k))
    _capi.check(status, "thm_wy_build_A")
    return A
