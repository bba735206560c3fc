"""The CPU oracle reproduces every committed golden fixture (tests/golden/*.npz):
guards the oracle against drift; the GPU side is tests/test_gpu_golden.py."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import conv as oconv
from oracle import deltanet as dn

GOLD = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLD / f"{name}.npz") as z:
        return {k: z[k].astype(np.float64) for k in z.files}


def close(a, b, rtol=1e-6, atol=1e-6):
    assert np.all(np.abs(a - b) <= atol + rtol * np.abs(b)), float(np.abs(a - b).max())


@pytest.mark.parametrize("name", ["conv_task0", "conv_task3", "conv_task4", "conv_bf16"])
def test_conv(name):
    d = load(name)
    close(oconv.causal_conv1d_numpy(d["x"], d["w"], d["b"], dtype=np.float64), d["out"])
    close(oconv.causal_conv1d_c(d["x"], d["w"], d["b"]), d["out"], 1e-5, 1e-5)


@pytest.mark.parametrize("name", ["wu_task0", "wu_bf16"])
def test_wu(name):
    d = load(name)
    w, u = dn.recompute_w_u_ref(d["k"], d["v"], d["beta"], d["A"], d["g"])
    close(w, d["w"])
    close(u, d["u"])


@pytest.mark.parametrize("name", ["o_task0", "o_bf16"])
def test_o(name):
    d = load(name)
    close(dn.chunk_fwd_o_ref(d["q"], d["k"], d["v"], d["g"], d["h"], float(d["scale"])), d["o"])


def test_h():
    d = load("h_ref")
    close(dn.chunk_fwd_h_ref(d["k"], d["v"], d["g"]), d["h"])
    d = load("h_delta_bf16")
    h, vn, S = dn.chunk_fwd_h_delta(d["k"], d["w"], d["u"], d["g"], h0=d["h0"])
    close(h, d["h"])
    close(vn, d["v_new"])
    close(S, d["ht"])


def test_chain():
    d = load("chain_bf16")
    o, S, _ = dn.chunk_gated_delta_forward(d["q"], d["k"], d["v"], d["beta"], d["g"], float(d["scale"]))
    close(o, d["o"])
    close(S, d["ht"])
