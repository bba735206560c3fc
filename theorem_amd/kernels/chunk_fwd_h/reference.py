"""Input generator and eager PyTorch references for the inter-chunk state
recurrence, with the interface of the reference's kernels/chunk_fwd_h/reference.py.

``generate_input`` follows reference.py:15-47 draw for draw (k, v = 0.5 N;
g = chunk-local cumsum of -0.05 U - 0.005) on a ``torch.Generator`` of
``device`` (the reference fixes "cuda:0"; the keyword lets the same draws run
on the CPU).  ``ref_kernel`` is reference.py:50-97 vectorised over (b, head):
h[c] is the state AFTER chunk c.  ``ref_kernel_delta`` is the delta-rule form
(h[c] BEFORE chunk c, v_new = u - w h, optional initial / final state).
"""
from __future__ import annotations

import torch

CHUNK_SIZE = 64


def generate_input(B: int, T: int, H: int, K: int, V: int, seed: int, device: str = "cuda:0",
                   dtype: torch.dtype = torch.float32):
    assert T % CHUNK_SIZE == 0, f"T={T} must be a multiple of CHUNK_SIZE={CHUNK_SIZE}"
    gen = torch.Generator(device=device).manual_seed(int(seed))
    k = torch.randn(B, T, H, K, generator=gen, dtype=torch.float32, device=device) * 0.5
    v = torch.randn(B, T, H, V, generator=gen, dtype=torch.float32, device=device) * 0.5
    g_inc = -0.05 * torch.rand(B, T, H, generator=gen, dtype=torch.float32, device=device) - 0.005
    NT = T // CHUNK_SIZE
    g = torch.cumsum(g_inc.view(B, NT, CHUNK_SIZE, H), dim=2).reshape(B, T, H).contiguous()
    return {"k": k.to(dtype), "v": v.to(dtype), "g": g, "B": B, "T": T, "H": H, "K": K, "V": V}


def _chunked(x, B, NT, H):
    return x.float().reshape(B, NT, CHUNK_SIZE, H, *x.shape[3:]).transpose(2, 3)  # [B, NT, H, BT, ...]


def ref_kernel(data) -> torch.Tensor:
    k, v, g = data["k"], data["v"], data["g"]
    B, T, H = k.shape[:3]
    K, V = k.shape[-1], v.shape[-1]
    NT = T // CHUNK_SIZE
    kc, vc, gc = _chunked(k, B, NT, H), _chunked(v, B, NT, H), _chunked(g, B, NT, H)
    h = torch.zeros(B, NT, H, K, V, device=k.device, dtype=torch.float32)
    state = torch.zeros(B, H, K, V, device=k.device, dtype=torch.float32)
    for c in range(NT):
        g_end = gc[:, c, :, -1]
        v_gated = vc[:, c] * torch.exp(g_end.unsqueeze(-1) - gc[:, c]).unsqueeze(-1)
        state = state * torch.exp(g_end)[..., None, None] + kc[:, c].transpose(-1, -2).contiguous() @ v_gated.contiguous()
        h[:, c] = state
    return h


def ref_kernel_delta(data):
    """Returns (h [B,NT,H,K,V] fp32, v_new [B,T,H,V] fp32, final state [B,H,K,V] fp32)."""
    k, w, u, g = data["k"], data["w"], data["u"], data.get("g")
    B, T, H = k.shape[:3]
    K, V = k.shape[-1], u.shape[-1]
    NT = T // CHUNK_SIZE
    kc, wc, uc = _chunked(k, B, NT, H), _chunked(w, B, NT, H), _chunked(u, B, NT, H)
    gc = _chunked(g, B, NT, H) if g is not None else torch.zeros(B, NT, H, CHUNK_SIZE, device=k.device)
    h0 = data.get("initial_state")
    S = torch.zeros(B, H, K, V, device=k.device) if h0 is None else h0.float().clone()
    h = torch.zeros(B, NT, H, K, V, device=k.device)
    vn = torch.zeros(B, NT, H, CHUNK_SIZE, V, device=k.device)
    for c in range(NT):
        h[:, c] = S
        vn[:, c] = uc[:, c] - wc[:, c] @ S
        gl = gc[:, c, :, -1]
        kg = kc[:, c] * torch.exp(gl.unsqueeze(-1) - gc[:, c]).unsqueeze(-1)
        S = S * torch.exp(gl)[..., None, None] + kg.transpose(-1, -2).contiguous() @ vn[:, c].contiguous()
    return h, vn.transpose(2, 3).reshape(B, T, H, V), S
