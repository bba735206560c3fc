"""The eager PyTorch baselines of theorem_amd/benchmarks/pytorch_baseline.py
(the vectorised forms of the reference's benchmarks/pytorch_baseline.py:121-229)
against the CPU oracle, and the baseline script itself on the GPU.

CPU tests: each eager form, run on CPU tensors (fp32), equals the oracle's
float64 restatement of the same op at 1e-4.  GPU tests: for one benchmark
shape per kernel, the HIP kernel and the eager form agree at the task
tolerance (1e-2), and the script's main() (timer of
benchmarks/pytorch_baseline.py:72-96) writes one finite row per kernel.
"""
from __future__ import annotations

import csv
import math

import numpy as np
import pytest
import torch

from oracle import conv as oconv
from oracle import deltanet as odn
from tests.helpers import assert_close
from theorem_amd.benchmarks import pytorch_baseline as pb


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def test_conv_eager_matches_oracle():
    g = _gen(1)
    x, w, b = torch.randn(2, 16, 200, generator=g), torch.randn(16, 4, generator=g), torch.randn(16, generator=g)
    got = pb.conv_eager(x, w, b)
    assert_close(got, oconv.causal_conv1d_c(x.numpy(), w.numpy(), b.numpy()), 1e-4, 1e-4, "conv_eager")


def test_h_eager_matches_oracle():
    g = _gen(2)
    B, T, H, K, V = 2, 192, 3, 16, 8
    k, v = torch.randn(B, T, H, K, generator=g) * 0.5, torch.randn(B, T, H, V, generator=g) * 0.5
    gate = torch.cumsum((-0.05 * torch.rand(B, T, H, generator=g) - 0.005).reshape(B, T // 64, 64, H), 2)
    gate = gate.reshape(B, T, H).contiguous()
    got = pb.h_eager(k, v, gate)
    assert_close(got, odn.chunk_fwd_h_ref(k.double().numpy(), v.double().numpy(), gate.double().numpy()),
                 1e-4, 1e-4, "h_eager")


def test_o_eager_matches_oracle():
    g = _gen(3)
    B, T, H, K, V = 1, 128, 2, 16, 8
    q, k, v = (torch.randn(B, T, H, D, generator=g) for D in (K, K, V))
    gate = torch.cumsum((0.05 * torch.randn(B, T, H, generator=g)).reshape(B, T // 64, 64, H), 2)
    gate = gate.reshape(B, T, H).contiguous()
    h = torch.randn(B, T // 64, H, K, V, generator=g) * 0.1
    got = pb.o_eager(q, k, v, gate, h, 0.25)
    e = odn.chunk_fwd_o_ref(*(t.double().numpy() for t in (q, k, v, gate, h)), 0.25)
    assert_close(got, e, 1e-4, 1e-4, "o_eager")


def test_wu_eager_matches_oracle():
    g = _gen(4)
    B, T, H, K, V = 1, 128, 2, 16, 8
    k, v = torch.randn(B, T, H, K, generator=g) * 0.1, torch.randn(B, T, H, V, generator=g) * 0.1
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    gate = torch.cumsum((-0.05 * torch.rand(B, T, H, generator=g)).reshape(B, T // 64, 64, H), 2)
    gate = gate.reshape(B, T, H).contiguous()
    A = torch.from_numpy(odn.build_A(k.double().numpy(), beta.double().numpy(), gate.double().numpy())).float()
    w, u = pb.wu_eager(k, v, beta, A, gate)
    ew, eu = odn.recompute_w_u_ref(*(t.double().numpy() for t in (k, v, beta, A, gate)))
    assert_close(w, ew, 1e-4, 1e-4, "wu_eager w")
    assert_close(u, eu, 1e-4, 1e-4, "wu_eager u")


def test_main_refuses_without_gpu():
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    assert pb.main(["--no-compile", "--max-shapes", "1"]) == 2


@pytest.mark.gpu
@pytest.mark.parametrize("kname", pb.KERNELS)
def test_hip_and_eager_agree_on_a_benchmark_shape(kname):
    import yaml
    shape = yaml.safe_load((pb.PKG / "kernels" / kname / "task.yml").read_text())["shapes"]["benchmarks"][0]
    run_hip, run_eager, _ = pb._stage(kname, shape, False)
    a, b = run_hip(), run_eager()
    torch.cuda.synchronize()
    for x, y in zip(a if isinstance(a, tuple) else (a,), b if isinstance(b, tuple) else (b,)):
        assert_close(x, y, 1e-2, 1e-2, f"{kname} {shape}: HIP vs eager")


@pytest.mark.gpu
def test_baseline_script_main(tmp_path):
    out = tmp_path / "cmp.csv"
    assert pb.main(["--no-compile", "--max-shapes", "1", "--csv", str(out)]) == 0
    rows = list(csv.DictReader(out.open()))
    assert [r["kernel"] for r in rows] == pb.KERNELS
    for r in rows:
        assert math.isfinite(float(r["hip_min_us"])) and math.isfinite(float(r["eager_min_us"])), r
