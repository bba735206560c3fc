"""Gated DeltaNet chunk forward composed from the three HIP kernels.

    A      = (I + strict_lower(beta_i (k_i . k_j) e^{g_i - g_j}))^{-1}   per 64-token chunk
    (w, u) = recompute_w_u(k, v, beta, A, g)                            HIP
    (h, v_new, S) = chunk_fwd_h delta form (h[c] before chunk c)        HIP
    o      = chunk_fwd_o(q, k, v_new, g, h, scale)                      HIP
    (for bf16 the last three in one kernel from A, chunk_fwd_fused_a, which
    never forms w and u; or the first two in one kernel, wy_fwd, and the last
    two in another, chunk_fwd_fused)

The reference never composes its ops (each is tested alone); this is the
forward of chunked Gated DeltaNet that the three ops are the stages of, and
it reproduces the token-by-token gated delta rule
    S_t = e^{a_t} S_{t-1};  S_t += beta_t k_t (v_t - S_t^T k_t)^T;  o_t = scale S_t^T q_t
with g the chunk-local cumsum of a.

``build_A`` (the WY matrix) is the HIP kernel thm_wy_build_A; ``wy_fwd`` is
thm_wy_fwd.
"""
from __future__ import annotations

import torch

from .kernels import _capi, chunk_fwd_h, chunk_fwd_o, recompute_w_u

BT = 64


def chunk_local_cumsum(a: torch.Tensor, logsigmoid: bool = False) -> torch.Tensor:
    """g [B, T, H] fp32: per 64-token chunk, the inclusive cumsum of a (or of
    log(sigmoid(a)) with ``logsigmoid``), on the GPU (thm_chunk_local_cumsum)."""
    B, T, H = a.shape
    assert T % BT == 0, f"T={T} must be a multiple of {BT}"
    _capi.require_device(a)
    code = _capi.dtype_code(a, "a")
    a = _capi.prep(a, "a")
    g = torch.empty(B, T, H, dtype=torch.float32, device=a.device)
    status = _capi.load_library().thm_chunk_local_cumsum(
        _capi.ptr(a), _capi.ptr(g), B, T, H, BT, code, 1 if logsigmoid else 0, _capi.stream_of(a))
    _capi.check(status, "thm_chunk_local_cumsum")
    return g


def build_A(k: torch.Tensor, beta: torch.Tensor, g: torch.Tensor | None) -> torch.Tensor:
    """A [B, T, H, 64] fp32 = per-chunk (I + strict_lower(beta_i k_i.k_j e^{g_i - g_j}))^{-1} (HIP)."""
    return recompute_w_u.build_A(k, beta, g, sign=+1)


def wy_fwd(k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor, g: torch.Tensor | None,
           sign: int = +1) -> tuple[torch.Tensor, torch.Tensor]:
    """(w, u) = recompute_w_u(k, v, beta, A, g) with A = build_A(k, beta, g, sign)
    formed inside the same HIP kernel and never written (thm_wy_fwd; bf16 k, v)."""
    B, T, H, K = k.shape
    V = v.shape[-1]
    assert T % BT == 0, f"T={T} must be a multiple of {BT}"
    assert v.shape[:3] == (B, T, H) and beta.shape == (B, T, H) and (g is None or g.shape == (B, T, H))
    assert k.dtype == v.dtype == torch.bfloat16, "the fused path is bf16-only"
    _capi.require_device(k, v, beta, g)
    for name, t in (("beta", beta), ("g", g)):
        _capi.require_f32(t, name)
    k, v, beta, g = (_capi.prep(t, n) for t, n in ((k, "k"), (v, "v"), (beta, "beta"), (g, "g")))
    w = torch.empty_like(k)
    u = torch.empty_like(v)
    status = _capi.load_library().thm_wy_fwd(
        _capi.ptr(k), _capi.ptr(v), _capi.ptr(beta), _capi.ptr(g), _capi.ptr(w), _capi.ptr(u),
        B, T, H, K, V, BT, _capi.THM_DTYPE[torch.bfloat16], int(sign), _capi.stream_of(k))
    _capi.check(status, "thm_wy_fwd")
    return w, u


def chunk_fwd_fused(q, k, w, u, g, scale: float, initial_state=None, output_final_state: bool = False,
                    save_new_value: bool = False):
    """o (and optionally v_new, final state) of chunk_fwd_h (delta form) followed
    by chunk_fwd_o, in one HIP kernel that never writes the per-chunk states
    (thm_chunk_gated_delta_fwd; bf16 q, k, w, u).  Returns (o, v_new or None, ht or None)."""
    B, T, H, K = k.shape
    V = u.shape[-1]
    assert T % BT == 0, f"T={T} must be a multiple of {BT}"
    assert q.shape == k.shape == w.shape and u.shape[:3] == (B, T, H)
    assert q.dtype == k.dtype == w.dtype == u.dtype == torch.bfloat16, "the fused path is bf16-only"
    _capi.require_device(q, k, w, u, g, initial_state)
    for name, t in (("g", g), ("initial_state", initial_state)):
        _capi.require_f32(t, name)
    q, k, w, u, g, h0 = (_capi.prep(t, n) for t, n in ((q, "q"), (k, "k"), (w, "w"), (u, "u"), (g, "g"),
                                                       (initial_state, "initial_state")))
    o = torch.empty_like(u)
    vn = torch.empty_like(u) if save_new_value else None
    ht = torch.empty(B, H, K, V, dtype=torch.float32, device=k.device) if output_final_state else None
    status = _capi.load_library().thm_chunk_gated_delta_fwd(
        _capi.ptr(q), _capi.ptr(k), _capi.ptr(w), _capi.ptr(u), _capi.ptr(g), _capi.ptr(h0), _capi.ptr(o),
        _capi.ptr(vn), _capi.ptr(ht), float(scale), B, T, H, K, V, BT, _capi.THM_DTYPE[torch.bfloat16],
        _capi.stream_of(k))
    _capi.check(status, "thm_chunk_gated_delta_fwd")
    return o, vn, ht


def chunk_fwd_fused_a(q, k, v, beta, A, g, scale: float, initial_state=None, output_final_state: bool = False,
                      save_new_value: bool = False):
    """The same as chunk_fwd_fused from the WY matrix A instead of w and u:
    v_new = A (beta (v - e^g k S)) = u - w S per chunk, in one HIP kernel
    (thm_chunk_gated_delta_fwd_a; bf16 q, k, v; fp32 beta, A, g).  Returns
    (o, v_new or None, ht or None)."""
    B, T, H, K = k.shape
    V = v.shape[-1]
    assert T % BT == 0, f"T={T} must be a multiple of {BT}"
    assert q.shape == k.shape and v.shape[:3] == (B, T, H) and beta.shape == (B, T, H)
    assert A.shape == (B, T, H, BT) and (g is None or g.shape == (B, T, H))
    assert q.dtype == k.dtype == v.dtype == torch.bfloat16, "the fused path is bf16-only"
    _capi.require_device(q, k, v, beta, A, g, initial_state)
    for name, t in (("beta", beta), ("A", A), ("g", g), ("initial_state", initial_state)):
        _capi.require_f32(t, name)
    q, k, v, beta, A, g, h0 = (_capi.prep(t, n) for t, n in ((q, "q"), (k, "k"), (v, "v"), (beta, "beta"),
                                                             (A, "A"), (g, "g"), (initial_state, "initial_state")))
    o = torch.empty_like(v)
    vn = torch.empty_like(v) if save_new_value else None
    ht = torch.empty(B, H, K, V, dtype=torch.float32, device=k.device) if output_final_state else None
    status = _capi.load_library().thm_chunk_gated_delta_fwd_a(
        _capi.ptr(q), _capi.ptr(k), _capi.ptr(v), _capi.ptr(beta), _capi.ptr(A), _capi.ptr(g), _capi.ptr(h0),
        _capi.ptr(o), _capi.ptr(vn), _capi.ptr(ht), float(scale), B, T, H, K, V, BT,
        _capi.THM_DTYPE[torch.bfloat16], _capi.stream_of(k))
    _capi.check(status, "thm_chunk_gated_delta_fwd_a")
    return o, vn, ht


def chunk_gated_delta_rule_fwd(q, k, v, beta, g, scale: float, initial_state=None,
                               output_final_state: bool = False, A: torch.Tensor | None = None,
                               return_intermediates: bool = False, a: torch.Tensor | None = None,
                               a_logsigmoid: bool = False, fused: bool | None = None,
                               fused_form: str = "A"):
    """o [B, T, H, V] (dtype of q) and the final state [B, H, K, V] fp32 (or None).

    bf16 inputs run fused kernels (``fused``, default for bf16 unless
    ``return_intermediates``, which needs w, u and the per-chunk states h):
    with ``fused_form`` "A" (default) build_A (unless ``A`` is given) and
    chunk_fwd_fused_a (w and u never formed: recurrence and output from A);
    with "wy" wy_fwd (A and w, u in one kernel; unless ``A`` is given) and
    chunk_fwd_fused.  Otherwise build_A, recompute_w_u, chunk_fwd_h,
    chunk_fwd_o.
    ``g`` is the chunk-local cumulative log decay [B, T, H] fp32 (or None: no
    gate).  Alternatively pass the per-token log decay ``a`` (g = None): g is
    then formed on the GPU by chunk_local_cumsum(a), of log(sigmoid(a)) when
    ``a_logsigmoid``."""
    B, T, H, K = k.shape
    V = v.shape[-1]
    if a is not None:
        assert g is None, "pass either g or a"
        g = chunk_local_cumsum(a, logsigmoid=a_logsigmoid)
    if fused is None:
        fused = k.dtype == torch.bfloat16 and not return_intermediates
    assert fused_form in ("A", "wy"), fused_form
    if fused and fused_form == "A":
        if A is None:
            A = build_A(k, beta, g)
        o, _, ht = chunk_fwd_fused_a(q, k, v, beta, A, g, scale, initial_state, output_final_state)
        return o, ht
    if fused and A is None:
        w, u = wy_fwd(k, v, beta, g, sign=+1)
    else:
        if A is None:
            A = build_A(k, beta, g)
        w, u = recompute_w_u.custom_kernel(recompute_w_u.Data(k=k, v=v, beta=beta, A=A, g=g,
                                                              B=B, T=T, H=H, K=K, V=V))
    if fused:
        o, _, ht = chunk_fwd_fused(q, k, w, u, g, scale, initial_state, output_final_state)
        return o, ht
    h, v_new, ht = chunk_fwd_h.custom_kernel(dict(k=k, w=w, u=u, g=g, initial_state=initial_state,
                                                  output_final_state=output_final_state))
    o = chunk_fwd_o.custom_kernel(dict(q=q, k=k, v=v_new, g=g, h=h, scale=scale))
    if return_intermediates:
        return o, ht, dict(A=A, g=g, w=w, u=u, h=h, v_new=v_new)
    return o, ht
