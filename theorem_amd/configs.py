"""Seeded input generators for the BASELINE.json configurations.

Every generator draws from ``torch.Generator('cpu').manual_seed(seed)`` in the
order listed in its docstring (so the same seed gives the same inputs on any
machine), then moves the tensors to ``device``.  ``N(0, s)`` means standard
deviation s.

Gate families (``gate=``):
  "logsigmoid" — g = chunk-local cumsum of logsigmoid(N(0,1))   (the configs)
  "mild"       — g = chunk-local cumsum of (-0.05 U(0,1) - 0.005) (the reference's
                 chunk_fwd_h generator, chunk_fwd_h/reference.py:39-45; keeps
                 exp(g_last) ~ 0.15 so the inter-chunk carry is visible)
  "zero"       — g = 0
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

BT = 64


def chunk_local_cumsum(a: torch.Tensor, bt: int = BT) -> torch.Tensor:
    B, T, H = a.shape
    return a.reshape(B, T // bt, bt, H).cumsum(dim=2).reshape(B, T, H).contiguous()


def make_gate(B: int, T: int, H: int, gen: torch.Generator, gate: str = "logsigmoid") -> torch.Tensor:
    """Chunk-local cumulative log gate g [B, T, H] fp32 (<= 0); one draw of B*T*H values."""
    if gate == "logsigmoid":
        a = F.logsigmoid(torch.randn(B, T, H, generator=gen))
    elif gate == "mild":
        a = -0.05 * torch.rand(B, T, H, generator=gen) - 0.005
    elif gate == "zero":
        a = torch.zeros(B, T, H)
    else:
        raise ValueError(f"unknown gate family {gate!r}")
    return chunk_local_cumsum(a)


def l2norm(x: torch.Tensor) -> torch.Tensor:
    return x / x.norm(dim=-1, keepdim=True).clamp_min(1e-12)


def build_A(k: torch.Tensor, beta: torch.Tensor, g: torch.Tensor, sign: int = +1,
            bt: int = BT) -> torch.Tensor:
    """A [B, T, H, bt] fp32 with A_c = (I + sign * M)^{-1},
    M = strict_lower(beta_i (k_i . k_j) e^{g_i - g_j}), computed in float64 on k's
    device from k as given (bf16 k is used exactly as rounded).  sign = -1 is the
    reference's (I - M)^{-1} (recompute_w_u/reference.py:48-91)."""
    B, T, H, K = k.shape
    NT = T // bt
    kc = k.double().reshape(B, NT, bt, H, K).permute(0, 1, 3, 2, 4)
    bc = beta.double().reshape(B, NT, bt, H).permute(0, 1, 3, 2)
    gc = g.double().reshape(B, NT, bt, H).permute(0, 1, 3, 2)
    M = (kc @ kc.transpose(-1, -2)) * bc.unsqueeze(-1) * torch.exp(gc.unsqueeze(-1) - gc.unsqueeze(-2))
    M = torch.tril(M, diagonal=-1)
    eye = torch.eye(bt, dtype=torch.float64, device=k.device).expand_as(M)
    Ac = torch.linalg.solve_triangular(eye + sign * M, eye, upper=False, unitriangular=True)
    return Ac.permute(0, 1, 3, 2, 4).reshape(B, T, H, bt).float().contiguous()


# --------------------------------------------------------------------------- conv

def make_conv_inputs(B: int, D: int, S: int, W: int, dtype: torch.dtype = torch.float32,
                     seed: int = 0, device="cpu"):
    """Config 0 / config 4 conv: draws x = N(0,1) [B,D,S], w = N(0,1)/2 [D,W],
    bias = N(0,0.1) [D], in that order, fp32, then cast to ``dtype``."""
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(B, D, S, generator=gen)
    w = torch.randn(D, W, generator=gen) / 2
    b = torch.randn(D, generator=gen) * 0.1
    return tuple(t.to(dtype).to(device).contiguous() for t in (x, w, b))


# --------------------------------------------------------------------------- DeltaNet ops

def make_wu_inputs(B=2, T=512, H=3, K=64, V=64, seed=0, device="cpu", dtype=torch.bfloat16,
                   gate="logsigmoid", sign=+1):
    """Config 1: draws k = N(0,1) [B,T,H,K] (L2-normalised over K), v = N(0,1) [B,T,H,V],
    beta_raw = N(0,1) [B,T,H] (beta = sigmoid), then the gate; k, v cast to ``dtype``;
    A from the rounded k in float64 (cast to fp32)."""
    gen = torch.Generator().manual_seed(seed)
    k = l2norm(torch.randn(B, T, H, K, generator=gen)).to(dtype)
    v = torch.randn(B, T, H, V, generator=gen).to(dtype)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    g = make_gate(B, T, H, gen, gate)
    A = build_A(k, beta, g, sign=sign)
    return {n: t.to(device).contiguous() for n, t in
            dict(k=k, v=v, beta=beta, A=A, g=g).items()}


def make_o_inputs(B=2, T=512, H=3, K=64, V=64, seed=0, device="cpu", dtype=torch.bfloat16,
                  gate="logsigmoid"):
    """Config 2: draws q, k = N(0,1) (L2-normalised), v = N(0,1), then the gate, then
    h = N(0,0.1) [B,T/64,H,K,V] fp32; scale = K^-1/2."""
    gen = torch.Generator().manual_seed(seed)
    q = l2norm(torch.randn(B, T, H, K, generator=gen)).to(dtype)
    k = l2norm(torch.randn(B, T, H, K, generator=gen)).to(dtype)
    v = torch.randn(B, T, H, V, generator=gen).to(dtype)
    g = make_gate(B, T, H, gen, gate)
    h = torch.randn(B, T // BT, H, K, V, generator=gen) * 0.1
    d = {n: t.to(device).contiguous() for n, t in dict(q=q, k=k, v=v, g=g, h=h).items()}
    d["scale"] = 1.0 / math.sqrt(K)
    return d


def make_h_inputs(B=2, T=1024, H=3, K=64, V=64, seed=0, device="cpu", dtype=torch.bfloat16,
                  gate="logsigmoid", h0_std: float = 0.0):
    """Config 3: draws k = N(0,1) (L2-normalised), w = N(0,0.1), u = N(0,0.1), then the
    gate, then (only if h0_std > 0) h0 = N(0,h0_std) [B,H,K,V] fp32; else h0 = None (zero)."""
    gen = torch.Generator().manual_seed(seed)
    k = l2norm(torch.randn(B, T, H, K, generator=gen)).to(dtype)
    w = (torch.randn(B, T, H, K, generator=gen) * 0.1).to(dtype)
    u = (torch.randn(B, T, H, V, generator=gen) * 0.1).to(dtype)
    g = make_gate(B, T, H, gen, gate)
    h0 = torch.randn(B, H, K, V, generator=gen) * h0_std if h0_std > 0 else None
    d = {n: t.to(device).contiguous() for n, t in dict(k=k, w=w, u=u, g=g).items()}
    d["h0"] = None if h0 is None else h0.to(device)
    return d


def make_chain_inputs(B=8, T=8192, H=16, K=128, V=128, seed=0, device="cpu",
                      dtype=torch.bfloat16, gate="logsigmoid"):
    """Config 4 chain: draws q, k = N(0,1) (L2-normalised), v = N(0,1), beta_raw = N(0,1),
    then the gate; A = (I + M)^{-1} built on ``device`` in float64."""
    gen = torch.Generator().manual_seed(seed)
    q = l2norm(torch.randn(B, T, H, K, generator=gen)).to(dtype)
    k = l2norm(torch.randn(B, T, H, K, generator=gen)).to(dtype)
    v = torch.randn(B, T, H, V, generator=gen).to(dtype)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    g = make_gate(B, T, H, gen, gate)
    d = {n: t.to(device).contiguous() for n, t in dict(q=q, k=k, v=v, beta=beta, g=g).items()}
    d["A"] = build_A(d["k"], d["beta"], d["g"], sign=+1)
    d["scale"] = 1.0 / math.sqrt(K)
    return d


@dataclass(frozen=True)
class ConfigSpec:
    name: str
    op: str
    shape: dict
    dtype: torch.dtype


CONFIGS = [
    ConfigSpec("cfg0", "causal_conv1d", dict(B=1, D=2560, S=4096, W=4), torch.float32),
    ConfigSpec("cfg1", "recompute_w_u", dict(B=2, T=512, H=3, K=64, V=64), torch.bfloat16),
    ConfigSpec("cfg2", "chunk_fwd_o", dict(B=2, T=512, H=3, K=64, V=64), torch.bfloat16),
    ConfigSpec("cfg3", "chunk_fwd_h", dict(B=2, T=1024, H=3, K=64, V=64), torch.bfloat16),
    ConfigSpec("cfg4", "chain", dict(B=8, T=8192, H=16, K=128, V=128), torch.bfloat16),
    ConfigSpec("cfg4", "causal_conv1d", dict(B=8, D=4096, S=8192, W=4), torch.bfloat16),
]
