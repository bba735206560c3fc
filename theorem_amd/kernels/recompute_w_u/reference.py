"""Input generator and eager PyTorch reference for the WY recompute, with the
interface of the reference's kernels/recompute_w_u/reference.py.

``generate_data`` follows reference.py:94-115 draw for draw on a CPU
``torch.Generator`` (k = 0.1 N, v = 0.1 N, beta = sigmoid(N), g = chunk
cumsum of -0.05 U), then builds A = (I - M)^{-1} (reference.py:48-91) with a
unit-triangular solve.  ``dtype`` casts k and v (beta, g and A stay fp32).
``ref_kernel`` computes u = A (v beta), w = A (k beta e^g) per chunk in fp32
(reference.py:118-149).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

BT = 64


@dataclass
class Data:
    k: torch.Tensor       # [B, T, H, K]
    v: torch.Tensor       # [B, T, H, V]
    beta: torch.Tensor    # [B, T, H]
    A: torch.Tensor       # [B, T, H, BT]
    g: torch.Tensor       # [B, T, H]
    B: int
    T: int
    H: int
    K: int
    V: int


def _build_A(k: torch.Tensor, beta: torch.Tensor, g: torch.Tensor) -> torch.Tensor:
    B, T, H, K = k.shape
    assert T % BT == 0, "T must be a multiple of BT (=64)"
    n = T // BT
    k_c = k.float().reshape(B, n, BT, H, K).permute(0, 1, 3, 2, 4)
    beta_c = beta.reshape(B, n, BT, H).permute(0, 1, 3, 2)
    g_c = g.reshape(B, n, BT, H).permute(0, 1, 3, 2)
    M = (k_c @ k_c.transpose(-1, -2)) * beta_c.unsqueeze(-1) * torch.exp(g_c.unsqueeze(-1) - g_c.unsqueeze(-2))
    M = torch.tril(M, diagonal=-1)
    eye = torch.eye(BT, device=k.device, dtype=torch.float32).expand_as(M)
    A_c = torch.linalg.solve_triangular(eye - M, eye, upper=False, unitriangular=True)
    return A_c.permute(0, 1, 3, 2, 4).reshape(B, T, H, BT).contiguous()


def generate_data(B: int, T: int, H: int, K: int, V: int, seed: int, device: str = "cuda",
                  dtype: torch.dtype = torch.float32) -> Data:
    gen = torch.Generator(device="cpu").manual_seed(seed)
    k = torch.randn(B, T, H, K, generator=gen, dtype=torch.float32) * 0.1
    v = torch.randn(B, T, H, V, generator=gen, dtype=torch.float32) * 0.1
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen, dtype=torch.float32))
    raw_g = -torch.rand(B, T, H, generator=gen, dtype=torch.float32) * 0.05
    assert T % BT == 0
    raw_g = raw_g.reshape(B, T // BT, BT, H).cumsum(dim=2).reshape(B, T, H)
    k, v, beta, raw_g = (t.to(device) for t in (k, v, beta, raw_g))
    A = _build_A(k, beta, raw_g)
    if dtype != torch.float32:
        k, v = k.to(dtype), v.to(dtype)
    return Data(k=k, v=v, beta=beta, A=A, g=raw_g, B=B, T=T, H=H, K=K, V=V)


def ref_kernel(data: Data) -> tuple[torch.Tensor, torch.Tensor]:
    k, v, beta, A, g = data.k.float(), data.v.float(), data.beta.float(), data.A.float(), data.g.float()
    B, T, H, K = k.shape
    V = v.shape[-1]
    n = T // BT
    k_c = k.reshape(B, n, BT, H, K).permute(0, 1, 3, 2, 4)
    v_c = v.reshape(B, n, BT, H, V).permute(0, 1, 3, 2, 4)
    beta_c = beta.reshape(B, n, BT, H).permute(0, 1, 3, 2)
    g_c = g.reshape(B, n, BT, H).permute(0, 1, 3, 2)
    A_c = A.reshape(B, n, BT, H, BT).permute(0, 1, 3, 2, 4).contiguous()
    u_c = A_c @ (v_c * beta_c.unsqueeze(-1)).contiguous()
    w_c = A_c @ (k_c * (beta_c * torch.exp(g_c)).unsqueeze(-1)).contiguous()
    u = u_c.permute(0, 1, 3, 2, 4).reshape(B, T, H, V).contiguous()
    w = w_c.permute(0, 1, 3, 2, 4).reshape(B, T, H, K).contiguous()
    return w, u


generate_input = generate_data
