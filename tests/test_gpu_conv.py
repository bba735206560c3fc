"""GPU parity of thm_causal_conv1d_fwd (through custom_kernel) against the CPU oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import conv as oconv
from tests.helpers import assert_close, bf16_round
from theorem_amd.kernels.causal_conv1d import custom_kernel, generate_input

pytestmark = pytest.mark.gpu

TASK_TESTS = [(1, 64, 64, 4, 4242), (2, 128, 128, 4, 5236), (1, 256, 256, 3, 1001),
              (1, 128, 64, 8, 5531), (4, 64, 128, 4, 9173)]


def _run(x, w, b, act=None):
    out = custom_kernel((x, w, b), activation=act)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("B,D,S,W,seed", TASK_TESTS)
def test_task_shapes_fp32(dev, B, D, S, W, seed):
    # The reference's task.yml test shapes; inputs from its generator (device RNG).
    x, w, b = generate_input(B, D, S, W, seed, device="cuda:0")
    out = _run(x, w, b)
    assert out.dtype == torch.float32 and out.shape == x.shape
    exp = oconv.causal_conv1d_c(x.cpu().numpy(), w.cpu().numpy(), b.cpu().numpy())
    assert_close(out, exp, 1e-4, 1e-4, "fp32 conv")


@pytest.mark.parametrize("W", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("S", [1, 3, 64, 255, 256, 1000, 1024, 3000])
def test_widths_and_lengths_fp32(dev, W, S):
    g = torch.Generator().manual_seed(S * 10 + W)
    x = torch.randn(2, 5, S, generator=g)
    w = torch.randn(5, W, generator=g) / 2
    b = torch.randn(5, generator=g) * 0.1
    out = _run(x.to(dev), w.to(dev), b.to(dev))
    assert_close(out, oconv.causal_conv1d_c(x.numpy(), w.numpy(), b.numpy()), 1e-4, 1e-4, f"W={W} S={S}")


@pytest.mark.parametrize("W", [2, 4, 8])
@pytest.mark.parametrize("S", [8, 512, 4096, 1000, 7])
def test_bf16(dev, W, S):
    g = torch.Generator().manual_seed(S + W)
    x = torch.randn(3, 6, S, generator=g).to(torch.bfloat16)
    w = (torch.randn(6, W, generator=g) / 2).to(torch.bfloat16)
    b = (torch.randn(6, generator=g) * 0.1).to(torch.bfloat16)
    out = _run(x.to(dev), w.to(dev), b.to(dev))
    assert out.dtype == torch.bfloat16
    exp = oconv.causal_conv1d_numpy(x.float().numpy(), w.float().numpy(), b.float().numpy(), dtype=np.float64)
    # fp32 accumulation, one bf16 rounding of the output.
    assert_close(out, exp, 1e-2, 1e-2, f"bf16 W={W} S={S}")
    assert np.abs(out.double().cpu().numpy() - bf16_round(exp)).max() <= np.abs(exp).max() * 2**-7


def test_mixed_dtypes_and_no_bias(dev):
    g = torch.Generator().manual_seed(7)
    x = torch.randn(2, 8, 640, generator=g)
    w = torch.randn(8, 4, generator=g).to(torch.bfloat16)
    out = _run(x.to(dev), w.to(dev), None)
    assert_close(out, oconv.causal_conv1d_numpy(x.numpy(), w.float().numpy(), None, dtype=np.float64),
                 1e-4, 1e-4, "fp32 x, bf16 w, no bias")


def test_silu(dev):
    g = torch.Generator().manual_seed(8)
    x, w, b = torch.randn(2, 16, 768, generator=g), torch.randn(16, 4, generator=g), torch.randn(16, generator=g)
    out = _run(x.to(dev), w.to(dev), b.to(dev), act="silu")
    exp = oconv.silu(oconv.causal_conv1d_numpy(x.numpy(), w.numpy(), b.numpy(), dtype=np.float64))
    assert_close(out, exp, 1e-4, 1e-4, "silu")


def test_unaligned_view_uses_scalar_path(dev):
    # A storage offset of one element breaks 16-byte alignment: the launcher
    # must fall back to per-element access and still be exact.
    g = torch.Generator().manual_seed(9)
    base = torch.randn(1 * 4 * 256 + 1, generator=g).to(dev)
    x = base[1:].view(1, 4, 256)
    w, b = torch.randn(4, 4, generator=g).to(dev), torch.randn(4, generator=g).to(dev)
    out = _run(x, w, b)
    assert_close(out, oconv.causal_conv1d_c(x.cpu().numpy(), w.cpu().numpy(), b.cpu().numpy()), 1e-4, 1e-4, "unaligned")


def test_empty_batch(dev):
    x = torch.empty(0, 4, 16, device=dev)
    out = _run(x, torch.randn(4, 4, device=dev), torch.randn(4, device=dev))
    assert out.shape == (0, 4, 16)


def test_cfg0_full_size(dev):
    # x[1,2560,4096] ~ N(0,1), w ~ N(0,1)/2, bias ~ N(0,0.1), fp32, seed 0.
    from theorem_amd.configs import make_conv_inputs
    x, w, b = make_conv_inputs(1, 2560, 4096, 4, torch.float32, seed=0, device=dev)
    out = _run(x, w, b)
    exp = oconv.causal_conv1d_c(x.cpu().numpy(), w.cpu().numpy(), b.cpu().numpy())
    assert_close(out, exp, 1e-4, 1e-4, "cfg0")
