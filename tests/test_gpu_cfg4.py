"""Parity at BASELINE.json's config 4, full size (the bench workload).

The full-size GPU results are checked four ways:
  * every output tensor of recompute_w_u, chunk_fwd_h and chunk_fwd_o against
    the CPU oracle in float32, one batch row at a time;
  * sampled slices against the CPU oracle (float64): whole sequences of
    sampled (batch, head) pairs for the state recurrence and the full chain
    (against the token-level gated delta rule), sampled chunks for
    recompute_w_u / chunk_fwd_o, sampled rows for the convolution; each
    kernel is fed the GPU's own upstream outputs, so a mismatch names the
    kernel;
  * the whole conv output against a plain PyTorch fp32 restatement on the GPU
    (elementwise tap sums, no library convolution);
  * homogeneity, which holds at any size: scaling the linear inputs by 2
    (exact in bf16 / fp32) must scale every output by exactly 2.
Tolerance rtol = atol = 1e-2 (bf16 inputs, the reference's task tolerance).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import conv as oconv
from oracle import deltanet as odn
from tests.helpers import assert_close
from theorem_amd import configs
from theorem_amd.kernels import causal_conv1d, chunk_fwd_h, chunk_fwd_o, recompute_w_u

pytestmark = pytest.mark.gpu

B, T, H, K, V = 8, 8192, 16, 128, 128
BT = 64
HEADS = [(0, 0), (7, 15), (3, 9)]                 # sampled (batch, head) pairs
CHUNKS = [(0, 0, 0), (7, 127, 15), (4, 63, 5)]    # sampled (batch, chunk, head) tiles


def np_(t):
    return t.detach().double().cpu().numpy()


def _homogeneous(out2, out, what):
    """out2 == 2 * out up to float rounding that scaling by 2 cannot cause
    (only a subnormal intermediate could break exactness)."""
    o, o2 = out.double(), out2.double()
    dev = float((o2 - 2 * o).abs().max())
    assert dev <= 1e-6 * float(o.abs().max()), f"{what}: not homogeneous, max dev {dev:.3e}"


@pytest.fixture(scope="module")
def chain(dev):
    print(f"[cfg4] chain inputs B={B} T={T} H={H} K={K} V={V} bf16", flush=True)
    d = configs.make_chain_inputs(B, T, H, K, V, seed=0, device=dev)
    w, u = recompute_w_u.custom_kernel(recompute_w_u.Data(k=d["k"], v=d["v"], beta=d["beta"], A=d["A"],
                                                          g=d["g"], B=B, T=T, H=H, K=K, V=V))
    h, vn, ht = chunk_fwd_h.custom_kernel(dict(k=d["k"], w=w, u=u, g=d["g"], output_final_state=True))
    o = chunk_fwd_o.custom_kernel(dict(q=d["q"], k=d["k"], v=vn, g=d["g"], h=h, scale=d["scale"]))
    torch.cuda.synchronize()
    d.update(w=w, u=u, h=h, vn=vn, ht=ht, o=o)
    return d


def _tile(t, b, c, hh):
    return t[b:b + 1, c * BT:(c + 1) * BT, hh:hh + 1]


def test_cfg4_recompute_w_u_sampled_chunks(chain):
    d = chain
    for b, c, hh in CHUNKS:
        ew, eu = odn.recompute_w_u_ref(*(np_(_tile(d[n], b, c, hh)) for n in ("k", "v", "beta", "A", "g")))
        assert_close(_tile(d["w"], b, c, hh), ew, 1e-2, 1e-2, f"w tile {(b, c, hh)}")
        assert_close(_tile(d["u"], b, c, hh), eu, 1e-2, 1e-2, f"u tile {(b, c, hh)}")


def test_cfg4_chunk_fwd_h_sampled_heads(chain):
    d = chain
    for b, hh in HEADS:
        sl = lambda t: t[b:b + 1, :, hh:hh + 1]  # noqa: E731
        eh, evn, eht = odn.chunk_fwd_h_delta(*(np_(sl(d[n])) for n in ("k", "w", "u", "g")))
        assert_close(d["h"][b:b + 1, :, hh:hh + 1], eh, 1e-2, 1e-2, f"h (b={b}, head={hh})")
        assert_close(sl(d["vn"]), evn, 1e-2, 1e-2, f"v_new (b={b}, head={hh})")
        assert_close(d["ht"][b:b + 1, hh:hh + 1], eht, 1e-2, 1e-2, f"final state (b={b}, head={hh})")


def test_cfg4_chunk_fwd_o_sampled_chunks(chain):
    d = chain
    for b, c, hh in CHUNKS:
        hc = d["h"][b:b + 1, c:c + 1, hh:hh + 1]
        eo = odn.chunk_fwd_o_diff(*(np_(_tile(d[n], b, c, hh)) for n in ("q", "k", "vn", "g")), np_(hc), d["scale"])
        assert_close(_tile(d["o"], b, c, hh), eo, 1e-2, 1e-2, f"o tile {(b, c, hh)}")


# Whole tensors at full size, one batch row at a time against the oracle in
# float32 (a few seconds per row on the host); each kernel is fed the GPU's own
# upstream outputs.
def _f32(t):
    return t.detach().float().cpu().numpy()


def test_cfg4_recompute_w_u_full(chain):
    d = chain
    for b in range(B):
        print(f"[cfg4] recompute_w_u full, batch row {b}", flush=True)
        ew, eu = odn.recompute_w_u_ref(*(_f32(d[n][b:b + 1]) for n in ("k", "v", "beta", "A", "g")),
                                       dtype=np.float32)
        assert_close(d["w"][b:b + 1], ew, 1e-2, 1e-2, f"w, batch row {b}")
        assert_close(d["u"][b:b + 1], eu, 1e-2, 1e-2, f"u, batch row {b}")


def test_cfg4_chunk_fwd_h_full(chain):
    d = chain
    for b in range(B):
        print(f"[cfg4] chunk_fwd_h full, batch row {b}", flush=True)
        eh, evn, eht = odn.chunk_fwd_h_delta(*(_f32(d[n][b:b + 1]) for n in ("k", "w", "u", "g")), dtype=np.float32)
        assert_close(d["h"][b:b + 1], eh, 1e-2, 1e-2, f"h, batch row {b}")
        assert_close(d["vn"][b:b + 1], evn, 1e-2, 1e-2, f"v_new, batch row {b}")
        assert_close(d["ht"][b:b + 1], eht, 1e-2, 1e-2, f"final state, batch row {b}")


def test_cfg4_chunk_fwd_o_full(chain):
    d = chain
    for b in range(B):
        print(f"[cfg4] chunk_fwd_o full, batch row {b}", flush=True)
        eo = odn.chunk_fwd_o_diff(*(_f32(d[n][b:b + 1]) for n in ("q", "k", "vn", "g", "h")), d["scale"],
                                  dtype=np.float32)
        assert_close(d["o"][b:b + 1], eo, 1e-2, 1e-2, f"o, batch row {b}")


def test_cfg4_chain_matches_token_recurrence(chain):
    # The whole 8192-token sequence of two sampled heads against the gated
    # delta rule run token by token.  The per-token log decay is recovered
    # from the chunk-local cumsum g (differences of fp32 values are exact in
    # float64, so its cumsum reproduces g).
    d = chain
    for b, hh in HEADS[:2]:
        sl = lambda t: np_(t[b:b + 1, :, hh:hh + 1])  # noqa: E731
        g = sl(d["g"])
        gc = g.reshape(1, T // BT, BT, 1)
        a = np.diff(gc, axis=2, prepend=0.0).reshape(1, T, 1)
        eo, eS = odn.gated_delta_rule_tokens(sl(d["q"]), sl(d["k"]), sl(d["v"]), sl(d["beta"]), a, d["scale"])
        assert_close(d["o"][b:b + 1, :, hh:hh + 1], eo, 1e-2, 1e-2, f"chain o (b={b}, head={hh})")
        assert_close(d["ht"][b:b + 1, hh:hh + 1], eS, 1e-2, 1e-2, f"chain final state (b={b}, head={hh})")


def test_cfg4_build_A_full(chain):
    # The HIP WY matrix over all 16384 chunks against the A of the input
    # generator (built per chunk in float64 on the GPU, then rounded to fp32).
    d = chain
    A = recompute_w_u.build_A(d["k"], d["beta"], d["g"], sign=+1)
    torch.cuda.synchronize()
    dev = float((A - d["A"]).abs().max())
    assert dev <= 1e-4 * float(d["A"].abs().max()), f"A max |diff| {dev:.3e}"


def test_cfg4_fused_forward(chain):
    # The fused h + o kernel at full size against the two separate kernels.
    from theorem_amd.chain import chunk_fwd_fused
    d = chain
    o, _, ht = chunk_fwd_fused(d["q"], d["k"], d["w"], d["u"], d["g"], d["scale"], None, True)
    torch.cuda.synchronize()
    for what, got, ref in (("o", o, d["o"]), ("final state", ht, d["ht"])):
        dev_ = float((got.float() - ref.float()).abs().max())
        assert dev_ <= 1e-2 * (1 + float(ref.float().abs().max())), f"fused {what}: max |diff| {dev_:.3e}"


def test_cfg4_fused_forward_a_full(chain):
    # The fused kernel's A form (v_new = A (beta (v - e^g k S)), w and u never
    # formed) at full size: every o, v_new and final-state element against the
    # separate kernels, and one sampled head's whole sequence against the
    # token-level gated delta rule.
    from theorem_amd.chain import chunk_fwd_fused_a
    d = chain
    o, vn, ht = chunk_fwd_fused_a(d["q"], d["k"], d["v"], d["beta"], d["A"], d["g"], d["scale"], None, True, True)
    torch.cuda.synchronize()
    for what, got, ref in (("o", o, d["o"]), ("v_new", vn, d["vn"]), ("final state", ht, d["ht"])):
        dev_ = float((got.float() - ref.float()).abs().max())
        assert dev_ <= 1e-2 * (1 + float(ref.float().abs().max())), f"A form {what}: max |diff| {dev_:.3e}"
    b, hh = HEADS[2]
    sl = lambda t: np_(t[b:b + 1, :, hh:hh + 1])  # noqa: E731
    a = np.diff(sl(d["g"]).reshape(1, T // BT, BT, 1), axis=2, prepend=0.0).reshape(1, T, 1)
    eo, eS = odn.gated_delta_rule_tokens(sl(d["q"]), sl(d["k"]), sl(d["v"]), sl(d["beta"]), a, d["scale"])
    assert_close(o[b:b + 1, :, hh:hh + 1], eo, 1e-2, 1e-2, f"A form o (b={b}, head={hh})")
    assert_close(ht[b:b + 1, hh:hh + 1], eS, 1e-2, 1e-2, f"A form final state (b={b}, head={hh})")


def test_cfg4_wy_fwd_full(chain):
    # The fused WY kernel at full size: bit-identical to A-builder + recompute_w_u
    # (the same fp32 A on chip), and within tolerance of the chain's w, u (whose A
    # is the generator's float64 inverse rounded to fp32).
    from theorem_amd.chain import wy_fwd
    d = chain
    w, u = wy_fwd(d["k"], d["v"], d["beta"], d["g"], sign=+1)
    A = recompute_w_u.build_A(d["k"], d["beta"], d["g"], sign=+1)
    w2, u2 = recompute_w_u.custom_kernel(recompute_w_u.Data(k=d["k"], v=d["v"], beta=d["beta"], A=A,
                                                            g=d["g"], B=B, T=T, H=H, K=K, V=V))
    torch.cuda.synchronize()
    assert torch.equal(w, w2) and torch.equal(u, u2), "wy_fwd differs from A-builder + recompute_w_u"
    for what, got, ref in (("w", w, d["w"]), ("u", u, d["u"])):
        dev_ = float((got.float() - ref.float()).abs().max())
        assert dev_ <= 1e-2 * (1 + float(ref.float().abs().max())), f"wy_fwd {what}: max |diff| {dev_:.3e}"


def test_cfg4_homogeneity(chain):
    # w, u are linear in A; h, v_new, final state are linear in u (zero initial
    # state); o is linear in (v, h) jointly.
    d = chain
    w2, u2 = recompute_w_u.custom_kernel(recompute_w_u.Data(k=d["k"], v=d["v"], beta=d["beta"], A=2 * d["A"],
                                                            g=d["g"], B=B, T=T, H=H, K=K, V=V))
    h2, vn2, ht2 = chunk_fwd_h.custom_kernel(dict(k=d["k"], w=d["w"], u=2 * d["u"], g=d["g"],
                                                  output_final_state=True))
    o2 = chunk_fwd_o.custom_kernel(dict(q=d["q"], k=d["k"], v=2 * d["vn"], g=d["g"], h=2 * d["h"],
                                        scale=d["scale"]))
    torch.cuda.synchronize()
    for out2, out, what in ((w2, d["w"], "w"), (u2, d["u"], "u"), (h2, d["h"], "h"), (vn2, d["vn"], "v_new"),
                            (ht2, d["ht"], "final state"), (o2, d["o"], "o")):
        _homogeneous(out2, out, what)


@pytest.fixture(scope="module")
def conv4(dev):
    print("[cfg4] conv inputs (8, 4096, 8192, W=4) bf16", flush=True)
    x, w, b = configs.make_conv_inputs(8, 4096, 8192, 4, dtype=torch.bfloat16, seed=0, device=dev)
    out = causal_conv1d.custom_kernel((x, w, b))
    torch.cuda.synchronize()
    return x, w, b, out


def test_cfg4_conv_full_vs_torch_fp32(conv4):
    x, w, b, out = conv4
    Wd = w.shape[1]
    S = x.shape[2]
    wf, bf = w.float(), b.float()
    for b0 in range(0, x.shape[0], 2):   # two batch rows at a time (fp32 temporaries of 0.27 GB each)
        xf = torch.nn.functional.pad(x[b0:b0 + 2].float(), (Wd - 1, 0))
        ref = bf[None, :, None].expand(xf.shape[0], -1, S).clone()
        for kk in range(Wd):
            ref += wf[None, :, kk, None] * xf[..., kk:kk + S]
        got = out[b0:b0 + 2].float()
        tol = 1e-2 + 1e-2 * ref.abs()
        bad = int(((got - ref).abs() > tol).sum())
        assert bad == 0, f"conv batch rows {b0}..{b0 + 1}: {bad} elements exceed 1e-2"


def test_cfg4_conv_sampled_rows_vs_oracle(conv4):
    x, w, b, out = conv4
    for bb, dd in [(0, 0), (7, 4095), (3, 1234)]:
        e = oconv.causal_conv1d_c(x[bb:bb + 1, dd:dd + 1].float().cpu().numpy(),
                                  w[dd:dd + 1].float().cpu().numpy(), b[dd:dd + 1].float().cpu().numpy())
        assert_close(out[bb:bb + 1, dd:dd + 1], e, 1e-2, 1e-2, f"conv row (b={bb}, d={dd})")


def test_cfg4_conv_homogeneity(conv4):
    x, w, b, out = conv4
    out2 = causal_conv1d.custom_kernel((2 * x, w, 2 * b))
    torch.cuda.synchronize()
    _homogeneous(out2, out, "conv")
