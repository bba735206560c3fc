"""Input generator and eager PyTorch reference for the causal conv, with the
interface of the reference's kernels/causal_conv1d/reference.py.

``generate_input`` draws x, weight, bias (in that order, all N(0,1) fp32) from a
``torch.Generator`` seeded per shape on the target device, as
reference.py:27-52 does; ``device`` is an added keyword (default "cuda:0", the
reference's fixed device) so the same draws can be made on the CPU.
``ref_kernel`` is ``F.pad`` + depthwise ``F.conv1d`` (reference.py:55-81),
computed in fp32 whatever the input dtype.
"""
from __future__ import annotations

from typing import Tuple

import torch
import torch.nn.functional as F

_DEVICE = "cuda:0"


def generate_input(B: int, D: int, S: int, W: int, seed: int, device: str = _DEVICE,
                   dtype: torch.dtype = torch.float32) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    gen = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn((B, D, S), device=device, dtype=torch.float32, generator=gen)
    weight = torch.randn((D, W), device=device, dtype=torch.float32, generator=gen)
    bias = torch.randn((D,), device=device, dtype=torch.float32, generator=gen)
    if dtype != torch.float32:
        x, weight, bias = x.to(dtype), weight.to(dtype), bias.to(dtype)
    return x, weight, bias


def ref_kernel(data, activation: str | None = None) -> torch.Tensor:
    x, weight, bias = data
    B, D, S = x.shape
    Dw, W = weight.shape
    assert D == Dw, f"channel mismatch: x has D={D}, weight has D={Dw}"
    assert bias is None or bias.shape == (D,), f"bias shape {tuple(bias.shape)} != ({D},)"
    xf = F.pad(x.float(), (W - 1, 0))
    out = F.conv1d(xf, weight.float().unsqueeze(1), bias=None if bias is None else bias.float(), groups=D)
    if activation == "silu":
        out = F.silu(out)
    assert out.shape == (B, D, S)
    return out.to(x.dtype)
