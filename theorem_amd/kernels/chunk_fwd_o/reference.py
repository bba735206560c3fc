"""Input generator and eager PyTorch reference for the chunkwise output, with
the interface of the reference's kernels/chunk_fwd_o/reference.py.

``_build_inputs`` / ``generate_input`` follow reference.py:36-77 draw for draw
on a CPU ``torch.Generator`` (q, k, v = N(0,1); g = 0.05 N; h = 0.1 N;
scale = K^-1/2).  ``dtype`` casts q, k, v (g and h stay fp32).
``ref_kernel`` evaluates reference.py:80-142 (factored gates q e^{g},
v e^{-g}, causal mask including the diagonal) vectorised over (b, chunk, head)
in fp32; the output has q's dtype.
"""
from __future__ import annotations

import math
from typing import Any, Dict

import torch

BT_DEFAULT = 64


def _build_inputs(B: int, T: int, H: int, K: int, V: int, seed: int, device: str = "cuda",
                  dtype: torch.dtype = torch.float32) -> Dict[str, Any]:
    gen = torch.Generator(device="cpu").manual_seed(int(seed))
    BT = BT_DEFAULT
    assert T % BT == 0, f"T={T} must be divisible by BT={BT}"
    NT = T // BT
    q = torch.randn(B, T, H, K, generator=gen, dtype=torch.float32)
    k = torch.randn(B, T, H, K, generator=gen, dtype=torch.float32)
    v = torch.randn(B, T, H, V, generator=gen, dtype=torch.float32)
    g = torch.randn(B, T, H, generator=gen, dtype=torch.float32) * 0.05
    h = torch.randn(B, NT, H, K, V, generator=gen, dtype=torch.float32) * 0.1
    q, k, v = (t.to(dtype).to(device) for t in (q, k, v))
    return {"q": q, "k": k, "v": v, "g": g.to(device), "h": h.to(device),
            "scale": 1.0 / math.sqrt(K), "B": B, "T": T, "H": H, "K": K, "V": V,
            "BT": BT, "NT": NT, "seed": seed}


def ref_kernel(data: Dict[str, Any]) -> torch.Tensor:
    q, k, v = data["q"].float(), data["k"].float(), data["v"].float()
    g, h = data["g"].float(), data["h"].float()
    scale = float(data["scale"])
    B, T, H, K = q.shape
    V = v.shape[-1]
    BT = int(data.get("BT", BT_DEFAULT))
    NT = T // BT
    q_c = q.reshape(B, NT, BT, H, K).permute(0, 1, 3, 2, 4)
    k_c = k.reshape(B, NT, BT, H, K).permute(0, 1, 3, 2, 4)
    v_c = v.reshape(B, NT, BT, H, V).permute(0, 1, 3, 2, 4)
    g_c = g.reshape(B, NT, BT, H).permute(0, 1, 3, 2)
    q_g = q_c * torch.exp(g_c).unsqueeze(-1)
    v_g = (v_c * torch.exp(-g_c).unsqueeze(-1)).contiguous()
    qk = q_g @ k_c.transpose(-1, -2).contiguous()
    idx = torch.arange(BT, device=q.device)
    qk = torch.where(idx.unsqueeze(0) <= idx.unsqueeze(1), qk, torch.zeros_like(qk))
    o = scale * (qk @ v_g + q_g @ h.contiguous())
    return o.permute(0, 1, 3, 2, 4).reshape(B, T, H, V).to(data["q"].dtype)


generate_input = _build_inputs
