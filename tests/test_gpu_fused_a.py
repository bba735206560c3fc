"""GPU parity of the fused forward from the WY matrix A
(thm_chunk_gated_delta_fwd_a, theorem_amd.chain.chunk_fwd_fused_a): per chunk
v_new = A (beta (v - e^g k S)), which equals u - w S for the recompute_w_u
outputs w = A (k beta e^g), u = A (v beta) (kernels/recompute_w_u/
reference.py:118-149), then the delta-form state recurrence
(kernels/chunk_fwd_h/kernel.py:61-138) and the output
(kernels/chunk_fwd_o/kernel.py:52-136) as in thm_chunk_gated_delta_fwd.

Checked against the float64 oracle (oracle/deltanet.py recompute_w_u_ref with
the same A, chunk_fwd_h_delta, chunk_fwd_o_diff) and against the w / u route
(recompute_w_u, then chunk_fwd_fused) on the same inputs.  Tolerance
rtol = atol = 1e-2 (bf16 q, k, v, o, v_new; the route through w and u rounds
w and u to bf16, this one does not).
"""
from __future__ import annotations

import pytest
import torch

from oracle import deltanet as odn
from tests.helpers import assert_close
from theorem_amd import chain, configs
from theorem_amd.kernels import recompute_w_u

pytestmark = pytest.mark.gpu


def np_(t):
    return None if t is None else t.detach().double().cpu().numpy()


def _inputs(B, T, H, K, V, gate, seed, dev, h0_std=0.1):
    gen = torch.Generator().manual_seed(seed)
    q = configs.l2norm(torch.randn(B, T, H, K, generator=gen)).to(torch.bfloat16)
    k = configs.l2norm(torch.randn(B, T, H, K, generator=gen)).to(torch.bfloat16)
    v = torch.randn(B, T, H, V, generator=gen).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    g = None if gate is None else configs.make_gate(B, T, H, gen, gate)
    h0 = torch.randn(B, H, K, V, generator=gen) * h0_std if h0_std > 0 else None
    to = lambda t: None if t is None else t.to(dev).contiguous()  # noqa: E731
    return to(q), to(k), to(v), to(beta), to(g), to(h0)


def _oracle(q, k, v, beta, A, g, h0, scale):
    gk = np_(g)
    ew, eu = odn.recompute_w_u_ref(np_(k), np_(v), np_(beta), np_(A), gk)
    eh, evn, eht = odn.chunk_fwd_h_delta(np_(k), ew, eu, gk, h0=np_(h0))
    return odn.chunk_fwd_o_diff(np_(q), np_(k), evn, gk, eh, scale), evn, eht


def _wu_route(q, k, v, beta, A, g, h0, scale):
    B, T, H, K = k.shape
    w, u = recompute_w_u.custom_kernel(recompute_w_u.Data(k=k, v=v, beta=beta, A=A, g=g, B=B, T=T, H=H, K=K,
                                                          V=v.shape[-1]))
    return chain.chunk_fwd_fused(q, k, w, u, g, scale, h0, True, True)


@pytest.mark.parametrize("K,V", [(64, 64), (64, 128), (128, 64), (128, 128)])
@pytest.mark.parametrize("gate", ["logsigmoid", "mild", None])
def test_fused_a_vs_oracle_and_wu_route(dev, K, V, gate):
    B, T, H = 2, 320, 3
    q, k, v, beta, g, h0 = _inputs(B, T, H, K, V, gate, 61, dev)
    scale = K ** -0.5
    A = chain.build_A(k, beta, g)
    o, vn, ht = chain.chunk_fwd_fused_a(q, k, v, beta, A, g, scale, h0, True, True)
    o2, vn2, ht2 = _wu_route(q, k, v, beta, A, g, h0, scale)
    torch.cuda.synchronize()
    assert o.dtype == torch.bfloat16 and o.shape == (B, T, H, V) and ht.shape == (B, H, K, V)
    what = f"K={K} V={V} gate={gate}"
    eo, evn, eht = _oracle(q, k, v, beta, A, g, h0, scale)
    assert_close(o, eo, 1e-2, 1e-2, f"o vs oracle {what}")
    assert_close(vn, evn, 1e-2, 1e-2, f"v_new vs oracle {what}")
    assert_close(ht, eht, 1e-2, 1e-2, f"final state vs oracle {what}")
    # About as accurate as the w / u route (which rounds w and u to bf16; this
    # form rounds t = beta (v - e^g k S) to bf16 before A).  Measured max errors
    # against the oracle: o 0.7-1.4x and the final state 0.8-1.2x the route's
    # (v_new, whose error is its own bf16 rounding, is held by the bar above).
    for name, a, b, e in (("o", o, o2, eo), ("final state", ht, ht2, eht)):
        err_a = float((a.double().cpu() - torch.from_numpy(e)).abs().max())
        err_wu = float((b.double().cpu() - torch.from_numpy(e)).abs().max())
        print(f"{what} {name}: max error A form {err_a:.3e}, w / u route {err_wu:.3e}")
        assert err_a <= 2 * err_wu + 1e-3, f"{name} {what}: A form {err_a:.3e} against the w / u route {err_wu:.3e}"
    # Optional outputs may be omitted (same o); T = 0 returns the initial state.
    o3, vn3, ht3 = chain.chunk_fwd_fused_a(q, k, v, beta, A, g, scale, h0)
    torch.cuda.synchronize()
    assert vn3 is None and ht3 is None and torch.equal(o3, o)
    e0 = torch.empty(B, 0, H, K, device=dev, dtype=torch.bfloat16)
    ev = torch.empty(B, 0, H, V, device=dev, dtype=torch.bfloat16)
    _, _, ht0 = chain.chunk_fwd_fused_a(e0, e0, ev, torch.empty(B, 0, H, device=dev),
                                        torch.empty(B, 0, H, 64, device=dev), None, scale, h0, True)
    torch.cuda.synchronize()
    assert torch.equal(ht0, h0)


@pytest.mark.parametrize("K,V", [(64, 64), (128, 128)])
@pytest.mark.parametrize("T", [64, 128, 192])
def test_fused_a_short_sequences(dev, K, V, T):
    # One to three chunks: the prologue and the clamped end-of-sequence loads
    # of the A / v tiles overlap.  Carry-visible gate and h0.
    B, H = 2, 3
    q, k, v, beta, g, h0 = _inputs(B, T, H, K, V, "mild", 63, dev)
    scale = K ** -0.5
    A = chain.build_A(k, beta, g)
    o, vn, ht = chain.chunk_fwd_fused_a(q, k, v, beta, A, g, scale, h0, True, True)
    torch.cuda.synchronize()
    eo, evn, eht = _oracle(q, k, v, beta, A, g, h0, scale)
    what = f"K={K} V={V} T={T}"
    assert_close(o, eo, 1e-2, 1e-2, f"o vs oracle {what}")
    assert_close(vn, evn, 1e-2, 1e-2, f"v_new vs oracle {what}")
    assert_close(ht, eht, 1e-2, 1e-2, f"final state vs oracle {what}")


def test_fused_a_long_mild_gate_carry(dev):
    # 64 chunks with a mild gate: the state carries across the whole sequence,
    # so a slip in the recurrence's v_new would accumulate.
    B, T, H, K, V = 1, 4096, 2, 128, 128
    q, k, v, beta, g, h0 = _inputs(B, T, H, K, V, "mild", 65, dev)
    scale = K ** -0.5
    A = chain.build_A(k, beta, g)
    o, vn, ht = chain.chunk_fwd_fused_a(q, k, v, beta, A, g, scale, h0, True, True)
    torch.cuda.synchronize()
    eo, evn, eht = _oracle(q, k, v, beta, A, g, h0, scale)
    assert_close(o, eo, 1e-2, 1e-2, "o vs oracle, 64 chunks")
    assert_close(ht, eht, 1e-2, 1e-2, "final state vs oracle, 64 chunks")


def test_driver_forms_agree(dev):
    # The driver's bf16 default (build_A + chunk_fwd_fused_a), its w / u form
    # (wy_fwd + chunk_fwd_fused) and its four-kernel form on the same inputs.
    gen = torch.Generator().manual_seed(67)
    B, T, H, K, V = 2, 256, 4, 128, 64
    q = configs.l2norm(torch.randn(B, T, H, K, generator=gen)).to(torch.bfloat16).to(dev)
    k = configs.l2norm(torch.randn(B, T, H, K, generator=gen)).to(torch.bfloat16).to(dev)
    v = torch.randn(B, T, H, V, generator=gen).to(torch.bfloat16).to(dev)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen)).to(dev)
    logits = torch.randn(B, T, H, generator=gen).to(dev)
    kw = dict(output_final_state=True, a=logits, a_logsigmoid=True)
    o1, s1 = chain.chunk_gated_delta_rule_fwd(q, k, v, beta, None, K ** -0.5, **kw)
    o2, s2 = chain.chunk_gated_delta_rule_fwd(q, k, v, beta, None, K ** -0.5, fused_form="wy", **kw)
    o3, s3 = chain.chunk_gated_delta_rule_fwd(q, k, v, beta, None, K ** -0.5, fused=False, **kw)
    torch.cuda.synchronize()
    assert_close(o1, o2, 1e-2, 1e-2, "driver o: A form vs w / u form")
    assert_close(s1, s2, 1e-2, 1e-2, "driver final state: A form vs w / u form")
    assert_close(o1, o3, 1e-2, 1e-2, "driver o: A form vs four kernels")
    assert_close(s1, s3, 1e-2, 1e-2, "driver final state: A form vs four kernels")
