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
    B, T, H, K = k.shape
    V = v.shape[-1]
    assert T % BT == 0, f"T={T} must be a multiple of {BT}"
    assert v.shape[:3] == (B, T, H) and beta.shape == (B, T, H) and A.shape == (B, T, H, BT)
    assert g is None or g.shape == (B, T, H)
    assert k.dtype == v.dtype, "k and v must share a dtype"
    _capi.require_device(k, v, beta, A, g)
    for name, t in (("beta", beta), ("A", A), ("g", g)):
        _capi.require_f32(t, name)
    code = _capi.dtype_code(k, "k")
    k, v, beta, A, g = (_capi.prep(t, n) for t, n in ((k, "k"), (v, "v"), (beta, "beta"), (A, "A"), (g, "g")))
    w = torch.empty_like(k)
    u = torch.empty_like(v)
    status = _capi.load_library().thm_recompute_w_u_fwd(
        _capi.ptr(k), _capi.ptr(v), _capi.ptr(beta), _capi.ptr(A), _capi.ptr(g), _capi.ptr(w), _capi.ptr(u),
        B, T, H, K, V, BT, code, _capi.stream_of(k))
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
