"""Gated DeltaNet chunk forward composed from the three HIP kernels.

    A      = (I + strict_lower(beta_i (k_i . k_j) e^{g_i - g_j}))^{-1}   per 64-token chunk
    (w, u) = recompute_w_u(k, v, beta, A, g)                            HIP
    (h, v_new, S) = chunk_fwd_h delta form (h[c] before chunk c)        HIP
    o      = chunk_fwd_o(q, k, v_new, g, h, scale)                      HIP

The reference never composes its ops (each is tested alone); this is the
forward of chunked Gated DeltaNet that the three ops are the stages of, and
it reproduces the token-by-token gated delta rule
    S_t = e^{a_t} S_{t-1};  S_t += beta_t k_t (v_t - S_t^T k_t)^T;  o_t = scale S_t^T q_t
with g the chunk-local cumsum of a.

``build_A`` is not one of the four kernels: it runs as batched torch ops on
the GPU (fp32 matmul + unit-triangular solve).
"""
from __future__ import annotations

import torch

from .kernels import chunk_fwd_h, chunk_fwd_o, recompute_w_u

BT = 64


def build_A(k: torch.Tensor, beta: torch.Tensor, g: torch.Tensor | None) -> torch.Tensor:
    """A [B, T, H, 64] fp32 = per-chunk (I + strict_lower(beta_i k_i.k_j e^{g_i - g_j}))^{-1}."""
    B, T, H, K = k.shape
    n = T // BT
    kc = k.float().reshape(B, n, BT, H, K).permute(0, 1, 3, 2, 4).contiguous()
    bc = beta.float().reshape(B, n, BT, H).permute(0, 1, 3, 2)
    M = (kc @ kc.transpose(-1, -2).contiguous()) * bc.unsqueeze(-1)
    if g is not None:
        gc = g.float().reshape(B, n, BT, H).permute(0, 1, 3, 2)
        M = M * torch.exp(gc.unsqueeze(-1) - gc.unsqueeze(-2))
    M = torch.tril(M, diagonal=-1)
    eye = torch.eye(BT, device=k.device, dtype=torch.float32).expand_as(M)
    Ac = torch.linalg.solve_triangular(eye + M, eye, upper=False, unitriangular=True)
    return Ac.permute(0, 1, 3, 2, 4).reshape(B, T, H, BT).contiguous()


def chunk_gated_delta_rule_fwd(q, k, v, beta, g, scale: float, initial_state=None,
                               output_final_state: bool = False, A: torch.Tensor | None = None,
                               return_intermediates: bool = False):
    """o [B, T, H, V] (dtype of q) and the final state [B, H, K, V] fp32 (or None)."""
    B, T, H, K = k.shape
    V = v.shape[-1]
    if A is None:
        A = build_A(k, beta, g)
    w, u = recompute_w_u.custom_kernel(recompute_w_u.Data(k=k, v=v, beta=beta, A=A, g=g, B=B, T=T, H=H, K=K, V=V))
    h, v_new, ht = chunk_fwd_h.custom_kernel(dict(k=k, w=w, u=u, g=g, initial_state=initial_state,
                                                  output_final_state=output_final_state))
    o = chunk_fwd_o.custom_kernel(dict(q=q, k=k, v=v_new, g=g, h=h, scale=scale))
    if return_intermediates:
        return o, ht, dict(A=A, w=w, u=u, h=h, v_new=v_new)
    return o, ht
