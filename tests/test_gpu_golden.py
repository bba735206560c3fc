"""The HIP kernels (through the drop-in wrappers) match the committed golden
fixtures: rtol = atol = 1e-2 for bf16 inputs, 1e-4 for the fp32 conv and
1e-3 for fp32 DeltaNet inputs."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from tests.helpers import assert_close
from theorem_amd.kernels import causal_conv1d, chunk_fwd_h, chunk_fwd_o, recompute_w_u

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"


def load(name, dtype=torch.float32):
    with np.load(GOLD / f"{name}.npz") as z:
        out = {}
        for k in z.files:
            a = z[k]
            out[k] = float(a) if a.ndim == 0 else a
    return out


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to("cuda:0")


@pytest.mark.parametrize("name,dtype,tol", [("conv_task0", torch.float32, 1e-4), ("conv_task3", torch.float32, 1e-4),
                                            ("conv_task4", torch.float32, 1e-4), ("conv_bf16", torch.bfloat16, 1e-2)])
def test_conv(name, dtype, tol):
    d = load(name)
    out = causal_conv1d.custom_kernel((dev(d["x"], dtype), dev(d["w"], dtype), dev(d["b"], dtype)))
    torch.cuda.synchronize()
    assert_close(out, d["out"], tol, tol, name)


@pytest.mark.parametrize("name,dtype,tol", [("wu_task0", torch.float32, 1e-3), ("wu_bf16", torch.bfloat16, 1e-2)])
def test_wu(name, dtype, tol):
    d = load(name)
    B, T, H, K = d["k"].shape
    V = d["v"].shape[-1]
    w, u = recompute_w_u.custom_kernel(recompute_w_u.Data(dev(d["k"], dtype), dev(d["v"], dtype), dev(d["beta"]),
                                                          dev(d["A"]), dev(d["g"]), B, T, H, K, V))
    torch.cuda.synchronize()
    assert_close(w, d["w"], tol, tol, name + " w")
    assert_close(u, d["u"], tol, tol, name + " u")


@pytest.mark.parametrize("name,dtype,tol", [("o_task0", torch.float32, 1e-3), ("o_bf16", torch.bfloat16, 1e-2)])
def test_o(name, dtype, tol):
    d = load(name)
    o = chunk_fwd_o.custom_kernel(dict(q=dev(d["q"], dtype), k=dev(d["k"], dtype), v=dev(d["v"], dtype),
                                       g=dev(d["g"]), h=dev(d["h"]), scale=d["scale"]))
    torch.cuda.synchronize()
    assert_close(o, d["o"], tol, tol, name)


def test_h():
    d = load("h_ref")
    h = chunk_fwd_h.custom_kernel(dict(k=dev(d["k"]), v=dev(d["v"]), g=dev(d["g"])))
    torch.cuda.synchronize()
    assert_close(h, d["h"], 1e-3, 1e-3, "h_ref")
    d = load("h_delta_bf16")
    h, vn, ht = chunk_fwd_h.custom_kernel(dict(k=dev(d["k"], torch.bfloat16), w=dev(d["w"], torch.bfloat16),
                                               u=dev(d["u"], torch.bfloat16), g=dev(d["g"]),
                                               initial_state=dev(d["h0"]), output_final_state=True))
    torch.cuda.synchronize()
    assert_close(h, d["h"], 1e-2, 1e-2, "h_delta h")
    assert_close(vn, d["v_new"], 1e-2, 1e-2, "h_delta v_new")
    assert_close(ht, d["ht"], 1e-2, 1e-2, "h_delta ht")


def test_chain():
    from theorem_amd.chain import chunk_gated_delta_rule_fwd
    d = load("chain_bf16")
    b16 = torch.bfloat16
    o, ht = chunk_gated_delta_rule_fwd(dev(d["q"], b16), dev(d["k"], b16), dev(d["v"], b16), dev(d["beta"]),
                                       dev(d["g"]), d["scale"], output_final_state=True)
    torch.cuda.synchronize()
    assert_close(o, d["o"], 1e-2, 1e-2, "chain o")
    assert_close(ht, d["ht"], 1e-2, 1e-2, "chain ht")
