"""GPU parity of the steps around the three DeltaNet kernels: the WY matrix
A (thm_wy_build_A, the reference's `_build_A`, recompute_w_u/reference.py:48-91)
and the gate preprocessing (thm_chunk_local_cumsum), against the CPU oracle
(float64), and of the chain driver that uses them.

Tolerances: A is fp32 from fp32 arithmetic (k k^T on MFMA is exact for bf16 k,
hi/lo split for fp32 k; fp32 forward substitution), held to 1e-4 relative to
max|A| against the float64 oracle; g is an fp32 running sum, held to 1e-5.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import deltanet as odn
from tests.helpers import assert_close
from theorem_amd import chain, configs
from theorem_amd.kernels import recompute_w_u

pytestmark = pytest.mark.gpu


def np_(t):
    return None if t is None else t.detach().double().cpu().numpy()


def _A_inputs(B, T, H, K, dtype, gate, seed, dev, normalize=True):
    gen = torch.Generator().manual_seed(seed)
    k = torch.randn(B, T, H, K, generator=gen)
    k = configs.l2norm(k) if normalize else 0.1 * k
    k = k.to(dtype)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    g = None if gate is None else configs.make_gate(B, T, H, gen, gate)
    return k.to(dev), beta.to(dev), (g.to(dev) if g is not None else None)


@pytest.mark.parametrize("K", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("sign", [1, -1])
@pytest.mark.parametrize("gate", ["logsigmoid", "mild", None])
def test_build_A_vs_oracle(dev, K, dtype, sign, gate):
    k, beta, g = _A_inputs(2, 256, 3, K, dtype, gate, seed=3, dev=dev)
    A = recompute_w_u.build_A(k, beta, g, sign=sign)
    torch.cuda.synchronize()
    assert A.dtype == torch.float32 and A.shape == (2, 256, 3, 64)
    gk = np_(g) if g is not None else np.zeros(tuple(k.shape[:3]))
    eA = odn.build_A(np_(k), np_(beta), gk, sign=sign)
    scale = np.abs(eA).max()
    assert_close(A, eA, 0, 1e-4 * scale, f"A K={K} {dtype} sign={sign} gate={gate}")
    # The defining identity, in float64 from the GPU's A: (I + sign M) A = I per chunk.
    Ab = np_(A).reshape(2, 4, 64, 3, 64).transpose(0, 1, 3, 2, 4)
    M = np.zeros_like(Ab)
    kc = np_(k).reshape(2, 4, 64, 3, K).transpose(0, 1, 3, 2, 4)
    bc = np_(beta).reshape(2, 4, 64, 3).transpose(0, 1, 3, 2)
    gc = gk.reshape(2, 4, 64, 3).transpose(0, 1, 3, 2)
    kk = kc @ np.swapaxes(kc, -1, -2)
    M = np.tril(kk * bc[..., None] * np.exp(gc[..., :, None] - gc[..., None, :]), -1)
    res = (np.eye(64) + sign * M) @ Ab - np.eye(64)
    assert np.abs(res).max() < 1e-4 * max(1.0, scale)


# bf16 grids of at least two tiles per persistent workgroup (4 per CU) run the
# software-pipelined A-builder: it must equal the one-tile kernel bit for bit
# (compared on a slice small enough to take the one-tile path) and the oracle.
@pytest.mark.parametrize("K", [64, 128])
@pytest.mark.parametrize("sign,gate", [(1, "logsigmoid"), (-1, "mild"), (1, None)])
def test_build_A_pipelined_path(dev, K, sign, gate):
    B, T, H = 2, 8192, 8
    k, beta, g = _A_inputs(B, T, H, K, torch.bfloat16, gate, seed=7, dev=dev)
    A = recompute_w_u.build_A(k, beta, g, sign=sign)
    sl = slice(T - 192, T)
    gs = None if g is None else g[1:, sl].contiguous()
    A1 = recompute_w_u.build_A(k[1:, sl].contiguous(), beta[1:, sl].contiguous(), gs, sign=sign)
    torch.cuda.synchronize()
    assert torch.equal(A[1:, sl], A1), f"pipelined A differs from the one-tile kernel (K={K} sign={sign})"
    kk = np_(k[:1, :128])
    gk = np_(g[:1, :128]) if g is not None else np.zeros((1, 128, H))
    eA = odn.build_A(kk, np_(beta[:1, :128]), gk, sign=sign)
    assert_close(A[:1, :128], eA, 0, 1e-4 * np.abs(eA).max(), f"A K={K} sign={sign} gate={gate}")


@pytest.mark.parametrize("K", [64, 128])
def test_build_A_pipelined_ragged_tail(dev, K):
    # 2049 tiles: one more than two per workgroup of the persistent grid (1024
    # on 256 CUs), so one workgroup takes a third tile.  Each chunk's A depends
    # on that chunk alone, so the whole tensor must equal the one-tile kernel's
    # over two slices that each stay under the pipelined path's threshold.
    B, T, H = 1, 64 * 683, 3
    k, beta, g = _A_inputs(B, T, H, K, torch.bfloat16, "logsigmoid", seed=8, dev=dev)
    A = recompute_w_u.build_A(k, beta, g, sign=1)
    cut = 64 * 600
    parts = [recompute_w_u.build_A(k[:, s].contiguous(), beta[:, s].contiguous(), g[:, s].contiguous(), sign=1)
             for s in (slice(0, cut), slice(cut, T))]
    torch.cuda.synchronize()
    assert torch.equal(A, torch.cat(parts, dim=1)), f"pipelined A (ragged tail) differs from the one-tile kernel, K={K}"


@pytest.mark.parametrize("B,T,H,K,V,seed", [(1, 64, 2, 64, 64, 4242), (2, 128, 4, 64, 64, 5236),
                                           (1, 256, 4, 64, 128, 1001)])
def test_build_A_matches_reference_generator(dev, B, T, H, K, V, seed):
    # The reference's own task.yml inputs (k = 0.1 N(0,1), not normalised; its sign):
    # the HIP A agrees with the A its generator builds with torch.
    data = recompute_w_u.generate_data(B, T, H, K, V, seed, device="cuda")
    A = recompute_w_u.build_A(data.k, data.beta, data.g, sign=-1)
    torch.cuda.synchronize()
    assert_close(A, data.A, 1e-4, 1e-5, "A vs generate_data")


def test_build_A_empty_and_errors(dev):
    k = torch.empty(1, 0, 2, 64, device=dev)
    A = recompute_w_u.build_A(k, torch.empty(1, 0, 2, device=dev), None, sign=1)
    torch.cuda.synchronize()
    assert A.shape == (1, 0, 2, 64)
    with pytest.raises(ValueError):
        recompute_w_u.build_A(torch.zeros(1, 64, 2, 96, device=dev), torch.zeros(1, 64, 2, device=dev), None)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("logsig", [False, True])
def test_chunk_local_cumsum(dev, dtype, logsig):
    gen = torch.Generator().manual_seed(7)
    a = (torch.randn(3, 320, 5, generator=gen) * 3).to(dtype)
    g = chain.chunk_local_cumsum(a.to(dev), logsigmoid=logsig)
    torch.cuda.synchronize()
    x = np_(a)
    e = odn.chunk_local_cumsum(odn.logsigmoid(x) if logsig else x)
    assert_close(g, e, 1e-5, 1e-5, f"g {dtype} logsigmoid={logsig}")
    g0 = chain.chunk_local_cumsum(torch.empty(3, 0, 5, device=dev, dtype=dtype), logsigmoid=logsig)
    assert g0.shape == (3, 0, 5)


@pytest.mark.parametrize("K,V", [(64, 64), (128, 128)])
def test_chain_from_per_token_gates(dev, K, V):
    # The driver fed raw gate logits (g formed on the GPU as the chunk-local
    # cumsum of logsigmoid) equals the token-level gated delta rule.
    gen = torch.Generator().manual_seed(21)
    B, T, H = 1, 192, 2
    q = configs.l2norm(torch.randn(B, T, H, K, generator=gen)).to(torch.bfloat16)
    k = configs.l2norm(torch.randn(B, T, H, K, generator=gen)).to(torch.bfloat16)
    v = torch.randn(B, T, H, V, generator=gen).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    logits = torch.randn(B, T, H, generator=gen)
    scale = K ** -0.5
    o, ht, inter = chain.chunk_gated_delta_rule_fwd(q.to(dev), k.to(dev), v.to(dev), beta.to(dev), None, scale,
                                                    output_final_state=True, return_intermediates=True,
                                                    a=logits.to(dev), a_logsigmoid=True)
    torch.cuda.synchronize()
    a = odn.logsigmoid(np_(logits))
    assert_close(inter["g"], odn.chunk_local_cumsum(a), 1e-5, 1e-5, "g")
    eo, eS = odn.gated_delta_rule_tokens(np_(q), np_(k), np_(v), np_(beta), a, scale)
    assert_close(o, eo, 1e-2, 1e-2, "chain o")
    assert_close(ht, eS, 1e-2, 1e-2, "chain final state")


@pytest.mark.parametrize("K,V", [(64, 64), (64, 128), (128, 64), (128, 128)])
@pytest.mark.parametrize("gate", ["logsigmoid", None])
def test_fused_forward_matches_two_kernels_and_oracle(dev, K, V, gate):
    # chunk_fwd_fused = chunk_fwd_h (delta form) followed by chunk_fwd_o, without
    # the per-chunk states: against the two kernels and the float64 oracle.
    from theorem_amd.kernels import chunk_fwd_h, chunk_fwd_o
    B, T, H = 2, 320, 3
    d = configs.make_h_inputs(B, T, H, K, V, seed=31, device=dev, dtype=torch.bfloat16,
                              gate=gate or "zero", h0_std=0.1)
    gen = torch.Generator().manual_seed(32)
    q = configs.l2norm(torch.randn(B, T, H, K, generator=gen)).to(torch.bfloat16).to(dev)
    g = d["g"] if gate else None
    scale = K ** -0.5
    o, vn, ht = chain.chunk_fwd_fused(q, d["k"], d["w"], d["u"], g, scale, d["h0"], True, True)
    h, vn2, ht2 = chunk_fwd_h.custom_kernel(dict(k=d["k"], w=d["w"], u=d["u"], g=g, initial_state=d["h0"],
                                                 output_final_state=True))
    o2 = chunk_fwd_o.custom_kernel(dict(q=q, k=d["k"], v=vn2, g=g, h=h, scale=scale))
    torch.cuda.synchronize()
    assert o.dtype == torch.bfloat16 and o.shape == (B, T, H, V)
    assert_close(o, o2, 1e-2, 1e-2, f"fused o vs two kernels K={K} V={V} gate={gate}")
    assert_close(vn, vn2, 1e-2, 1e-2, "v_new")
    assert_close(ht, ht2, 1e-2, 1e-2, "final state")
    gk = np_(g) if g is not None else None
    eh, evn, eht = odn.chunk_fwd_h_delta(np_(d["k"]), np_(d["w"]), np_(d["u"]), gk, h0=np_(d["h0"]))
    eo = odn.chunk_fwd_o_diff(np_(q), np_(d["k"]), evn, gk, eh, scale)
    assert_close(o, eo, 1e-2, 1e-2, f"fused o vs oracle K={K} V={V} gate={gate}")
    assert_close(ht, eht, 1e-2, 1e-2, "final state vs oracle")
    # Optional outputs may be omitted; T = 0 returns the initial state.
    o3, vn3, ht3 = chain.chunk_fwd_fused(q, d["k"], d["w"], d["u"], g, scale, d["h0"])
    torch.cuda.synchronize()
    assert vn3 is None and ht3 is None and torch.equal(o3, o)
    e0 = torch.empty(B, 0, H, K, device=dev, dtype=torch.bfloat16)
    _, _, ht0 = chain.chunk_fwd_fused(e0, e0, e0, torch.empty(B, 0, H, V, device=dev, dtype=torch.bfloat16),
                                      None, scale, d["h0"], True)
    torch.cuda.synchronize()
    assert torch.equal(ht0, d["h0"])


@pytest.mark.parametrize("K,V", [(64, 64), (128, 128)])
@pytest.mark.parametrize("T", [64, 128, 192])
def test_fused_forward_short_sequences(dev, K, V, T):
    # One to three chunks: the fused kernel's prologue loads chunk 0 and the
    # w / u of chunk 1, and each chunk loads the w / u of the chunk two ahead,
    # so here the prologue and the end-of-sequence re-loads (chunk indices
    # clamped to the last chunk) overlap.  Carry-visible gate and h0, against
    # the two kernels and the float64 oracle.
    from theorem_amd.kernels import chunk_fwd_h, chunk_fwd_o
    B, H = 2, 3
    d = configs.make_h_inputs(B, T, H, K, V, seed=33, device=dev, dtype=torch.bfloat16, gate="mild", h0_std=0.1)
    gen = torch.Generator().manual_seed(34)
    q = configs.l2norm(torch.randn(B, T, H, K, generator=gen)).to(torch.bfloat16).to(dev)
    scale = K ** -0.5
    o, vn, ht = chain.chunk_fwd_fused(q, d["k"], d["w"], d["u"], d["g"], scale, d["h0"], True, True)
    h, vn2, ht2 = chunk_fwd_h.custom_kernel(dict(k=d["k"], w=d["w"], u=d["u"], g=d["g"], initial_state=d["h0"],
                                                 output_final_state=True))
    o2 = chunk_fwd_o.custom_kernel(dict(q=q, k=d["k"], v=vn2, g=d["g"], h=h, scale=scale))
    torch.cuda.synchronize()
    assert_close(o, o2, 1e-2, 1e-2, f"fused o vs two kernels K={K} T={T}")
    assert_close(vn, vn2, 1e-2, 1e-2, "v_new")
    assert_close(ht, ht2, 1e-2, 1e-2, "final state")
    gk = np_(d["g"])
    eh, evn, eht = odn.chunk_fwd_h_delta(np_(d["k"]), np_(d["w"]), np_(d["u"]), gk, h0=np_(d["h0"]))
    eo = odn.chunk_fwd_o_diff(np_(q), np_(d["k"]), evn, gk, eh, scale)
    assert_close(o, eo, 1e-2, 1e-2, f"fused o vs oracle K={K} T={T}")
    assert_close(vn, evn, 1e-2, 1e-2, "v_new vs oracle")
    assert_close(ht, eht, 1e-2, 1e-2, "final state vs oracle")


@pytest.mark.parametrize("K,V", [(64, 64), (64, 128), (128, 64), (128, 128)])
@pytest.mark.parametrize("sign", [1, -1])
@pytest.mark.parametrize("gate", ["logsigmoid", None])
def test_wy_fwd_matches_two_kernels_and_oracle(dev, K, V, sign, gate):
    # thm_wy_fwd = thm_wy_build_A followed by recompute_w_u with A kept on chip:
    # the same fp32 A and the same products, so w and u agree bit for bit; and
    # against the float64 oracle (A from the oracle's build_A).
    B, T, H = 2, 192, 3
    k, beta, g = _A_inputs(B, T, H, K, torch.bfloat16, gate, seed=41, dev=dev)
    gen = torch.Generator().manual_seed(42)
    v = torch.randn(B, T, H, V, generator=gen).to(torch.bfloat16).to(dev)
    w, u = chain.wy_fwd(k, v, beta, g, sign=sign)
    A = recompute_w_u.build_A(k, beta, g, sign=sign)
    w2, u2 = recompute_w_u.custom_kernel(recompute_w_u.Data(k=k, v=v, beta=beta, A=A, g=g, B=B, T=T, H=H, K=K, V=V))
    torch.cuda.synchronize()
    assert w.dtype == u.dtype == torch.bfloat16 and w.shape == k.shape and u.shape == v.shape
    assert torch.equal(w, w2), f"w differs from the two-kernel path (K={K} V={V} sign={sign} gate={gate})"
    assert torch.equal(u, u2), f"u differs from the two-kernel path (K={K} V={V} sign={sign} gate={gate})"
    gk = np_(g) if g is not None else np.zeros((B, T, H))
    eA = odn.build_A(np_(k), np_(beta), gk, sign=sign)
    ew, eu = odn.recompute_w_u_ref(np_(k), np_(v), np_(beta), eA, gk)
    assert_close(w, ew, 1e-2, 1e-2, f"w vs oracle K={K} V={V} sign={sign} gate={gate}")
    assert_close(u, eu, 1e-2, 1e-2, f"u vs oracle K={K} V={V} sign={sign} gate={gate}")


# Grids of at least two tiles per persistent workgroup (2 per CU: 1024 tiles on
# 256 CUs) run the software-pipelined WY kernel; these shapes force it at
# every K, V (both signs, with and without the gate).  1280 tiles: the
# workgroups get 2 or 3 tiles each.
@pytest.mark.parametrize("K,V", [(64, 64), (64, 128), (128, 64), (128, 128)])
@pytest.mark.parametrize("sign,gate", [(1, "logsigmoid"), (-1, None)])
def test_wy_fwd_pipelined_path(dev, K, V, sign, gate):
    B, T, H = 2, 8192, 5
    k, beta, g = _A_inputs(B, T, H, K, torch.bfloat16, gate, seed=43, dev=dev)
    gen = torch.Generator().manual_seed(44)
    v = torch.randn(B, T, H, V, generator=gen).to(torch.bfloat16).to(dev)
    w, u = chain.wy_fwd(k, v, beta, g, sign=sign)
    A = recompute_w_u.build_A(k, beta, g, sign=sign)
    w2, u2 = recompute_w_u.custom_kernel(recompute_w_u.Data(k=k, v=v, beta=beta, A=A, g=g, B=B, T=T, H=H, K=K, V=V))
    torch.cuda.synchronize()
    assert torch.equal(w, w2), f"w differs from the two-kernel path (K={K} V={V} sign={sign} gate={gate})"
    assert torch.equal(u, u2), f"u differs from the two-kernel path (K={K} V={V} sign={sign} gate={gate})"
    # The oracle on the first and last 64-token chunks of batch 0 (A is chunk-local).
    for t0 in (0, T - 64):
        sl = slice(t0, t0 + 64)
        kk, bb, vv = np_(k[:1, sl]), np_(beta[:1, sl]), np_(v[:1, sl])
        gk = np_(g[:1, sl]) if g is not None else np.zeros((1, 64, H))
        eA = odn.build_A(kk, bb, gk, sign=sign)
        ew, eu = odn.recompute_w_u_ref(kk, vv, bb, eA, gk)
        assert_close(w[:1, sl], ew, 1e-2, 1e-2, f"w vs oracle K={K} V={V} t0={t0}")
        assert_close(u[:1, sl], eu, 1e-2, 1e-2, f"u vs oracle K={K} V={V} t0={t0}")


def test_wy_fwd_empty_and_errors(dev):
    e = torch.empty(1, 0, 2, 64, device=dev, dtype=torch.bfloat16)
    w, u = chain.wy_fwd(e, e, torch.empty(1, 0, 2, device=dev), None)
    torch.cuda.synchronize()
    assert w.shape == (1, 0, 2, 64) and u.shape == (1, 0, 2, 64)
    z = torch.zeros(1, 64, 2, 96, device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        chain.wy_fwd(z, z, torch.zeros(1, 64, 2, device=dev), None)
    with pytest.raises(AssertionError):
        f = torch.zeros(1, 64, 2, 64, device=dev)
        chain.wy_fwd(f, f, torch.zeros(1, 64, 2, device=dev), None)


def test_driver_fused_matches_unfused(dev):
    # The driver's bf16 default (wy_fwd + chunk_fwd_fused) against its
    # four-kernel form on the same inputs.
    gen = torch.Generator().manual_seed(51)
    B, T, H, K, V = 2, 256, 4, 128, 64
    q = configs.l2norm(torch.randn(B, T, H, K, generator=gen)).to(torch.bfloat16).to(dev)
    k = configs.l2norm(torch.randn(B, T, H, K, generator=gen)).to(torch.bfloat16).to(dev)
    v = torch.randn(B, T, H, V, generator=gen).to(torch.bfloat16).to(dev)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen)).to(dev)
    logits = torch.randn(B, T, H, generator=gen).to(dev)
    o1, s1 = chain.chunk_gated_delta_rule_fwd(q, k, v, beta, None, K ** -0.5, output_final_state=True,
                                              a=logits, a_logsigmoid=True)
    o2, s2 = chain.chunk_gated_delta_rule_fwd(q, k, v, beta, None, K ** -0.5, output_final_state=True,
                                              a=logits, a_logsigmoid=True, fused=False)
    torch.cuda.synchronize()
    assert_close(o1, o2, 1e-2, 1e-2, "driver o fused vs unfused")
    assert_close(s1, s2, 1e-2, 1e-2, "driver final state fused vs unfused")
