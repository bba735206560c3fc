"""Writes the golden fixtures in this directory: small seeded inputs and the
float64 oracle outputs for each hot-path kernel (plus the composed chain),
stored together so parity does not depend on RNG streams of a given torch or
NumPy version.

    python tests/golden/make_golden.py

Draw orders: reference-shape cases follow the reference's own generators on a
CPU generator (kernels/recompute_w_u/reference.py:94-115,
kernels/chunk_fwd_o/reference.py:36-77; the conv case uses
scripts/cpu_reference.py:31-37's NumPy generator); config-style cases use
theorem_amd.configs at reduced sizes.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

from oracle import conv as oconv  # noqa: E402
from oracle import deltanet as dn  # noqa: E402
from theorem_amd import configs  # noqa: E402


def f64(t):
    return t.double().cpu().numpy() if isinstance(t, torch.Tensor) else np.asarray(t, dtype=np.float64)


def f32(t):
    return t.float().cpu().numpy() if isinstance(t, torch.Tensor) else np.asarray(t, dtype=np.float32)


def save(name, **arrays):
    # float64 oracle outputs are stored as float32 (fixtures are compared at
    # >= 1e-6 relative; float32 keeps the files small)
    arrays = {k: (v.astype(np.float32) if v.dtype == np.float64 and v.ndim else v) for k, v in arrays.items()}
    np.savez_compressed(HERE / f"{name}.npz", **arrays)
    print(f"{name}: " + ", ".join(f"{k}{tuple(v.shape)}" for k, v in arrays.items()))


def main():
    # causal_conv1d: reference task.yml test shapes 0, 3, 4, NumPy draws of cpu_reference.py:31-37
    for i, (B, D, S, W, seed) in [(0, (1, 64, 64, 4, 4242)), (3, (1, 128, 64, 8, 5531)), (4, (4, 64, 128, 4, 9173))]:
        rng = np.random.default_rng(seed)
        x = rng.standard_normal((B, D, S), dtype=np.float32)
        w = rng.standard_normal((D, W), dtype=np.float32)
        b = rng.standard_normal((D,), dtype=np.float32)
        save(f"conv_task{i}", x=x, w=w, b=b, out=oconv.causal_conv1d_numpy(x, w, b, dtype=np.float64))
    x, w, b = configs.make_conv_inputs(2, 64, 512, 4, torch.bfloat16, seed=7)
    save("conv_bf16", x=f32(x), w=f32(w), b=f32(b), out=oconv.causal_conv1d_numpy(f64(x), f64(w), f64(b), dtype=np.float64))

    # recompute_w_u
    from theorem_amd.kernels.recompute_w_u import generate_data
    d = generate_data(1, 64, 2, 64, 64, 4242, device="cpu")
    ww, uu = dn.recompute_w_u_ref(*(f64(t) for t in (d.k, d.v, d.beta, d.A, d.g)))
    save("wu_task0", k=f32(d.k), v=f32(d.v), beta=f32(d.beta), A=f32(d.A), g=f32(d.g), w=ww, u=uu)
    d = configs.make_wu_inputs(1, 128, 2, 64, 128, seed=8)
    ww, uu = dn.recompute_w_u_ref(*(f64(d[n]) for n in ("k", "v", "beta", "A", "g")))
    save("wu_bf16", **{n: f32(d[n]) for n in ("k", "v", "beta", "A", "g")}, w=ww, u=uu)

    # chunk_fwd_o
    from theorem_amd.kernels.chunk_fwd_o import generate_input as o_gen
    d = o_gen(1, 64, 1, 64, 64, 4242, device="cpu")
    o = dn.chunk_fwd_o_ref(*(f64(d[n]) for n in ("q", "k", "v", "g", "h")), d["scale"])
    save("o_task0", **{n: f32(d[n]) for n in ("q", "k", "v", "g", "h")}, scale=np.float64(d["scale"]), o=o)
    d = configs.make_o_inputs(1, 128, 2, 64, 128, seed=9, gate="mild")
    o = dn.chunk_fwd_o_diff(*(f64(d[n]) for n in ("q", "k", "v", "g", "h")), d["scale"])
    save("o_bf16", **{n: f32(d[n]) for n in ("q", "k", "v", "g", "h")}, scale=np.float64(d["scale"]), o=o)

    # chunk_fwd_h: reference form (reference.py:15-47 distributions, CPU generator) and delta form
    from theorem_amd.kernels.chunk_fwd_h import generate_input as h_gen
    d = h_gen(1, 128, 2, 64, 64, 4242, device="cpu")
    save("h_ref", k=f32(d["k"]), v=f32(d["v"]), g=f32(d["g"]), h=dn.chunk_fwd_h_ref(f64(d["k"]), f64(d["v"]), f64(d["g"])))
    d = configs.make_h_inputs(1, 256, 2, 64, 64, seed=10, gate="mild", h0_std=0.1)
    h, vn, S = dn.chunk_fwd_h_delta(*(f64(d[n]) for n in ("k", "w", "u", "g")), h0=f64(d["h0"]))
    save("h_delta_bf16", **{n: f32(d[n]) for n in ("k", "w", "u", "g", "h0")}, h=h, v_new=vn, ht=S)

    # chain: token-level gated delta rule
    gen = torch.Generator().manual_seed(11)
    B, T, H, K, V = 1, 128, 2, 64, 64
    q = configs.l2norm(torch.randn(B, T, H, K, generator=gen)).to(torch.bfloat16)
    k = configs.l2norm(torch.randn(B, T, H, K, generator=gen)).to(torch.bfloat16)
    v = torch.randn(B, T, H, V, generator=gen).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    a = -0.05 * torch.rand(B, T, H, generator=gen) - 0.005
    g = configs.chunk_local_cumsum(a)
    eo, eS = dn.gated_delta_rule_tokens(f64(q), f64(k), f64(v), f64(beta), f64(a), K ** -0.5)
    save("chain_bf16", q=f32(q), k=f32(k), v=f32(v), beta=f32(beta), a=f32(a), g=f32(g),
         scale=np.float64(K ** -0.5), o=eo, ht=eS)


if __name__ == "__main__":
    main()
