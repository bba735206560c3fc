"""Pins the NumPy DeltaNet oracle (oracle/deltanet.py) to the mathematics:
closed forms, library routines (torch / LAPACK), per-token brute-force loops and
the token-level gated delta rule.  Each check is chosen so that a plausible
slip (dropped decay, wrong diagonal, wrong sign of M, pre- vs post-update
storage) fails it; test_mutations_are_caught plants such slips in oracle copies."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import deltanet as dn

RNG = np.random.default_rng(1234)


def rand(*shape, scale=1.0):
    return RNG.standard_normal(shape) * scale


def gate(B, T, H, kind="mild"):
    if kind == "zero":
        a = np.zeros((B, T, H))
    elif kind == "mild":
        a = -0.05 * RNG.random((B, T, H)) - 0.005
    else:
        a = np.log(1.0 / (1.0 + np.exp(-RNG.standard_normal((B, T, H)))))
    return a, dn.chunk_local_cumsum(a)


def l2n(x):
    return x / np.linalg.norm(x, axis=-1, keepdims=True)


# --------------------------------------------------------------------------- chunk_fwd_h

def h_bruteforce_ref(k, v, g):
    """Per-token loops: S after chunk c = sum over tokens t <= end of c of
    exp(g_end(c') - g_t + sum_{c'' in (c', c]} g_end(c'')) k_t v_t^T, t in chunk c'."""
    B, T, H, K = k.shape
    V = v.shape[-1]
    NT = T // 64
    out = np.zeros((B, NT, H, K, V))
    for b in range(B):
        for h in range(H):
            gend = [g[b, 64 * c + 63, h] for c in range(NT)]
            for c in range(NT):
                S = np.zeros((K, V))
                for cp in range(c + 1):
                    for t in range(64 * cp, 64 * cp + 64):
                        dec = gend[cp] - g[b, t, h] + sum(gend[cpp] for cpp in range(cp + 1, c + 1))
                        S += np.exp(dec) * np.outer(k[b, t, h], v[b, t, h])
                out[b, c, h] = S
    return out


def test_h_ref_bruteforce_and_closed_forms():
    B, T, H, K, V = 1, 192, 2, 8, 4
    k, v = rand(B, T, H, K), rand(B, T, H, V)
    _, g = gate(B, T, H, "mild")
    h = dn.chunk_fwd_h_ref(k, v, g)
    assert np.abs(h - h_bruteforce_ref(k, v, g)).max() < 1e-10
    # NT = 1: h[0] = k^T (v e^{g_end - g}).
    h1 = dn.chunk_fwd_h_ref(k[:, :64], v[:, :64], g[:, :64])
    e = np.einsum("bthk,bthv->bhkv", k[:, :64], v[:, :64] * np.exp(g[:, 63:64] - g[:, :64])[..., None])
    assert np.abs(h1[:, 0] - e).max() < 1e-12
    # g = 0: prefix sums of per-chunk k^T v.
    h0 = dn.chunk_fwd_h_ref(k, v, np.zeros_like(g))
    per = np.stack([np.einsum("bthk,bthv->bhkv", k[:, 64 * c:64 * c + 64], v[:, 64 * c:64 * c + 64]) for c in range(3)], 1)
    assert np.abs(h0 - np.cumsum(per, axis=1)).max() < 1e-10
    # k = 0 -> h = 0; linearity in v.
    assert np.abs(dn.chunk_fwd_h_ref(np.zeros_like(k), v, g)).max() == 0
    v2 = rand(B, T, H, V)
    lin = dn.chunk_fwd_h_ref(k, 2 * v + v2, g) - 2 * h - dn.chunk_fwd_h_ref(k, v2, g)
    assert np.abs(lin).max() < 1e-10


def test_h_ref_matches_torch_restatement():
    from theorem_amd.kernels.chunk_fwd_h import ref_kernel
    B, T, H, K, V = 2, 128, 3, 16, 8
    k, v = rand(B, T, H, K), rand(B, T, H, V)
    _, g = gate(B, T, H, "mild")
    t = lambda x: torch.from_numpy(x).float()  # noqa: E731
    got = ref_kernel(dict(k=t(k), v=t(v), g=t(g))).double().numpy()
    assert np.abs(got - dn.chunk_fwd_h_ref(k, v, g)).max() < 1e-4


def test_h_delta_reduces_to_reference_form():
    B, T, H, K, V = 1, 256, 2, 16, 8
    k, u = rand(B, T, H, K), rand(B, T, H, V)
    _, g = gate(B, T, H, "mild")
    h0 = rand(B, H, K, V)
    hd, vn, S = dn.chunk_fwd_h_delta(k, np.zeros_like(k), u, g, h0=h0)
    # with w = 0 the delta form is the reference form seeded with h0 and stored
    # one chunk earlier (state before, not after, each chunk)
    href = dn.chunk_fwd_h_ref(k, u, g)
    decay = np.exp(np.stack([g[:, 64 * c + 63] for c in range(4)], 1).cumsum(1))  # [B, NT, H]
    href0 = href + decay[..., None, None] * h0[:, None]
    assert np.abs(hd[:, 0] - h0).max() == 0
    assert np.abs(hd[:, 1:] - href0[:, :-1]).max() < 1e-10
    assert np.abs(S - href0[:, -1]).max() < 1e-10
    assert np.array_equal(vn, u)


def test_h_delta_bruteforce_single_head():
    # explicit per-chunk recurrence with plain loops (one head, small sizes)
    T, K, V = 128, 4, 3
    k, w, u = rand(1, T, 1, K), rand(1, T, 1, K), rand(1, T, 1, V)
    _, g = gate(1, T, 1, "mild")
    h, vn, S = dn.chunk_fwd_h_delta(k, w, u, g)
    St = np.zeros((K, V))
    for c in range(2):
        assert np.abs(h[0, c, 0] - St).max() < 1e-12
        gl = g[0, 64 * c + 63, 0]
        new = np.zeros((K, V))
        for t in range(64 * c, 64 * c + 64):
            vt = u[0, t, 0] - w[0, t, 0] @ St
            assert np.abs(vn[0, t, 0] - vt).max() < 1e-12
            new += np.exp(gl - g[0, t, 0]) * np.outer(k[0, t, 0], vt)
        St = np.exp(gl) * St + new
    assert np.abs(S[0, 0] - St).max() < 1e-12


def test_h_delta_matches_torch_restatement():
    from theorem_amd.kernels.chunk_fwd_h import ref_kernel_delta
    B, T, H, K, V = 1, 192, 2, 16, 8
    k, w, u = rand(B, T, H, K), rand(B, T, H, K, scale=0.1), rand(B, T, H, V)
    _, g = gate(B, T, H, "logsigmoid")
    t = lambda x: torch.from_numpy(x).float()  # noqa: E731
    h, vn, S = ref_kernel_delta(dict(k=t(k), w=t(w), u=t(u), g=t(g)))
    eh, evn, eS = dn.chunk_fwd_h_delta(k, w, u, g)
    assert np.abs(h.double().numpy() - eh).max() < 1e-4
    assert np.abs(vn.double().numpy() - evn).max() < 1e-4
    assert np.abs(S.double().numpy() - eS).max() < 1e-4


# --------------------------------------------------------------------------- chunk_fwd_o

def o_bruteforce(q, k, v, g, h, scale):
    B, T, H, K = q.shape
    V = v.shape[-1]
    o = np.zeros((B, T, H, V))
    for b in range(B):
        for hh in range(H):
            for i in range(T):
                c = i // 64
                acc = np.exp(g[b, i, hh]) * (q[b, i, hh] @ h[b, c, hh])
                for j in range(64 * c, i + 1):  # causal, diagonal included
                    acc = acc + (q[b, i, hh] @ k[b, j, hh]) * np.exp(g[b, i, hh] - g[b, j, hh]) * v[b, j, hh]
                o[b, i, hh] = scale * acc
    return o


def test_o_bruteforce_and_forms():
    B, T, H, K, V = 1, 128, 2, 8, 4
    q, k, v = rand(B, T, H, K), rand(B, T, H, K), rand(B, T, H, V)
    _, g = gate(B, T, H, "mild")
    h = rand(B, T // 64, H, K, V, scale=0.1)
    ref = dn.chunk_fwd_o_ref(q, k, v, g, h, 0.3)
    assert np.abs(ref - o_bruteforce(q, k, v, g, h, 0.3)).max() < 1e-10
    assert np.abs(dn.chunk_fwd_o_diff(q, k, v, g, h, 0.3) - ref).max() < 1e-10


def test_o_closed_forms_and_torch():
    from theorem_amd.kernels.chunk_fwd_o import ref_kernel
    B, T, H, K, V = 2, 128, 2, 16, 8
    q, k, v = rand(B, T, H, K), rand(B, T, H, K), rand(B, T, H, V)
    _, g = gate(B, T, H, "logsigmoid")
    h = rand(B, T // 64, H, K, V, scale=0.1)
    # h = 0, g = 0: scale * tril_incl(q k^T) v per chunk (torch.tril + matmul).
    o = dn.chunk_fwd_o_ref(q, k, v, np.zeros_like(g), np.zeros_like(h), 0.5)
    qc = torch.from_numpy(q).reshape(B, 2, 64, H, K).permute(0, 1, 3, 2, 4)
    kc = torch.from_numpy(k).reshape(B, 2, 64, H, K).permute(0, 1, 3, 2, 4)
    vc = torch.from_numpy(v).reshape(B, 2, 64, H, V).permute(0, 1, 3, 2, 4)
    e = 0.5 * torch.tril(qc @ kc.transpose(-1, -2)) @ vc
    assert np.abs(o - e.permute(0, 1, 3, 2, 4).reshape(B, T, H, V).numpy()).max() < 1e-10
    # v = 0: scale e^g q h[c].
    o2 = dn.chunk_fwd_o_diff(q, k, np.zeros_like(v), g, h, 0.5)
    e2 = 0.5 * np.exp(g)[..., None] * np.einsum("bchtk,bchkv->bchtv", np.moveaxis(q.reshape(B, 2, 64, H, K), 3, 2),
                                                  np.moveaxis(h, 2, 2)).transpose(0, 1, 3, 2, 4).reshape(B, T, H, V)
    assert np.abs(o2 - e2).max() < 1e-10
    t = lambda x: torch.from_numpy(x).float()  # noqa: E731
    got = ref_kernel(dict(q=t(q), k=t(k), v=t(v), g=t(g), h=t(h), scale=0.5)).double().numpy()
    assert np.abs(got - dn.chunk_fwd_o_ref(q, k, v, g, h, 0.5)).max() < 1e-3


# --------------------------------------------------------------------------- recompute_w_u / A

def test_build_A_inverse_and_solver():
    B, T, H, K = 1, 128, 2, 16
    k = l2n(rand(B, T, H, K))
    beta = 1 / (1 + np.exp(-rand(B, T, H)))
    _, g = gate(B, T, H, "logsigmoid")
    for sign in (-1, +1):
        A = dn.build_A(k, beta, g, sign=sign)
        kc = k.reshape(B, 2, 64, H, K)
        for c in range(2):
            for h in range(H):
                kk = kc[0, c, :, h]
                gg = g[0, 64 * c:64 * c + 64, h]
                M = np.tril(beta[0, 64 * c:64 * c + 64, h, None] * (kk @ kk.T) * np.exp(gg[:, None] - gg[None, :]), -1)
                Ac = A[0, 64 * c:64 * c + 64, h]
                assert np.abs((np.eye(64) + sign * M) @ Ac - np.eye(64)).max() < 1e-10
                # library routine: unit-lower-triangular solve
                ref = torch.linalg.solve_triangular(torch.from_numpy(np.eye(64) + sign * M), torch.eye(64, dtype=torch.float64),
                                                    upper=False, unitriangular=True).numpy()
                assert np.abs(Ac - ref).max() < 1e-10


def test_recompute_w_u_identity_and_torch():
    from theorem_amd.kernels.recompute_w_u import Data, ref_kernel
    B, T, H, K, V = 1, 128, 2, 16, 8
    k, v = l2n(rand(B, T, H, K)), rand(B, T, H, V)
    beta = 1 / (1 + np.exp(-rand(B, T, H)))
    _, g = gate(B, T, H, "mild")
    eye = np.tile(np.eye(64), (2, 1))[None, :, None, :].repeat(H, axis=2)
    w, u = dn.recompute_w_u_ref(k, v, beta, eye, g)
    assert np.abs(w - k * (beta * np.exp(g))[..., None]).max() < 1e-12
    assert np.abs(u - v * beta[..., None]).max() < 1e-12
    A = dn.build_A(k, beta, g, sign=-1)
    t = lambda x: torch.from_numpy(x).float()  # noqa: E731
    rw, ru = ref_kernel(Data(t(k), t(v), t(beta), t(A), t(g), B, T, H, K, V))
    ew, eu = dn.recompute_w_u_ref(k, v, beta, A, g)
    assert np.abs(rw.double().numpy() - ew).max() < 1e-4
    assert np.abs(ru.double().numpy() - eu).max() < 1e-4


def test_ut_residual():
    # (I + M) u = beta v for the gated-delta-rule A (checks A without inverting again)
    B, T, H, K, V = 1, 64, 1, 16, 8
    k, v = l2n(rand(B, T, H, K)), rand(B, T, H, V)
    beta = 1 / (1 + np.exp(-rand(B, T, H)))
    _, g = gate(B, T, H, "logsigmoid")
    A = dn.build_A(k, beta, g, sign=+1)
    _, u = dn.recompute_w_u_ref(k, v, beta, A, g)
    kk, gg, bb = k[0, :, 0], g[0, :, 0], beta[0, :, 0]
    M = np.tril(bb[:, None] * (kk @ kk.T) * np.exp(gg[:, None] - gg[None, :]), -1)
    assert np.abs((np.eye(64) + M) @ u[0, :, 0] - bb[:, None] * v[0, :, 0]).max() < 1e-10


# --------------------------------------------------------------------------- chain

@pytest.mark.parametrize("kind", ["logsigmoid", "mild", "zero"])
def test_chain_equals_token_recurrence(kind):
    B, T, H, K, V = 1, 192, 2, 16, 8
    q, k, v = l2n(rand(B, T, H, K)), l2n(rand(B, T, H, K)), rand(B, T, H, V)
    beta = 1 / (1 + np.exp(-rand(B, T, H)))
    a, g = gate(B, T, H, kind)
    h0 = rand(B, H, K, V, scale=0.1)
    o, S, _ = dn.chunk_gated_delta_forward(q, k, v, beta, g, 0.25, h0=h0)
    eo, eS = dn.gated_delta_rule_tokens(q, k, v, beta, a, 0.25, h0=h0)
    assert np.abs(o - eo).max() < 1e-10
    assert np.abs(S - eS).max() < 1e-10


def test_mutations_are_caught():
    """Plausible slips planted in copies of the oracle fail the pins above."""
    B, T, H, K, V = 1, 128, 1, 8, 4
    q, k, v = rand(B, T, H, K), rand(B, T, H, K), rand(B, T, H, V)
    _, g = gate(B, T, H, "mild")
    h = rand(B, 2, H, K, V, scale=0.1)
    good = o_bruteforce(q, k, v, g, h, 0.3)
    # 1. exclusive diagonal in the causal mask
    qc, kc, vc = (dn._chunks(x, 64, np.float64) for x in (q, k, v))
    gc = dn._chunks(g, 64, np.float64)
    hc = np.moveaxis(h, 2, 1)
    strict = np.tril(np.ones((64, 64), dtype=bool), -1)
    P = (qc @ np.swapaxes(kc, -1, -2)) * np.exp(np.where(strict, gc[..., :, None] - gc[..., None, :], -np.inf))
    bad = dn._unchunk(0.3 * (P @ vc + np.exp(gc)[..., None] * (qc @ hc)))
    assert np.abs(bad - good).max() > 1e-3
    # 2. dropped decay on the carried state (chunk_fwd_h)
    href = dn.chunk_fwd_h_ref(k, v, g)
    kc_, vc_ = dn._chunks(k, 64, np.float64), dn._chunks(v, 64, np.float64)
    S = np.zeros((B, H, K, V))
    bad_h = []
    for c in range(2):
        gend = gc[:, :, c, -1]
        S = S + np.swapaxes(kc_[:, :, c], -1, -2) @ (vc_[:, :, c] * np.exp(gend[..., None] - gc[:, :, c])[..., None])
        bad_h.append(S.copy())
    assert np.abs(np.stack(bad_h, 1) - href).max() > 1e-4
    assert np.abs(href - h_bruteforce_ref(k, v, g)).max() < 1e-10
    # 3. wrong sign of M in A: the chain no longer matches the token recurrence
    beta = 1 / (1 + np.exp(-rand(B, T, H)))
    a, g2 = gate(B, T, H, "zero")
    kn = l2n(k)
    A_bad = dn.build_A(kn, beta, g2, sign=-1)
    o_bad, _, _ = dn.chunk_gated_delta_forward(q, kn, v, beta, g2, 0.25)
    w, u = dn.recompute_w_u_ref(kn, v, beta, A_bad, g2)
    hh, vn, _ = dn.chunk_fwd_h_delta(kn, w, u, g2)
    o_bad = dn.chunk_fwd_o_diff(q, kn, vn, g2, hh, 0.25)
    eo, _ = dn.gated_delta_rule_tokens(q, kn, v, beta, a, 0.25)
    assert np.abs(o_bad - eo).max() > 1e-3


# --------------------------------------------------------------------------- gates

def test_chunk_local_cumsum_pins():
    # Brute-force loop; constant increment closed form a * (t % 64 + 1); the
    # sum restarts at every chunk; first differences inside a chunk give a back.
    a = rand(2, 192, 3)
    g = dn.chunk_local_cumsum(a)
    ref = np.zeros_like(a)
    for b in range(2):
        for h in range(3):
            run = 0.0
            for t in range(192):
                run = a[b, t, h] if t % 64 == 0 else run + a[b, t, h]
                ref[b, t, h] = run
    np.testing.assert_allclose(g, ref, rtol=1e-12, atol=1e-12)
    c = dn.chunk_local_cumsum(np.full((1, 128, 1), -0.25))
    np.testing.assert_allclose(c[0, :, 0], -0.25 * (np.arange(128) % 64 + 1))
    assert np.all(g[:, ::64] == a[:, ::64])
    d = np.diff(g.reshape(2, 3, 64, 3), axis=2)
    np.testing.assert_allclose(d, a.reshape(2, 3, 64, 3)[:, :, 1:], atol=1e-12)


def test_logsigmoid_pins():
    # torch's library routine, logsigmoid(0) = -log 2, the tails (-> 0 and -> x),
    # and logsigmoid(x) - logsigmoid(-x) = x.
    x = np.linspace(-60, 60, 4001)
    np.testing.assert_allclose(dn.logsigmoid(x), torch.nn.functional.logsigmoid(torch.from_numpy(x)).numpy(),
                               rtol=1e-12, atol=1e-12)
    assert abs(dn.logsigmoid(np.array([0.0]))[0] + np.log(2.0)) < 1e-15
    np.testing.assert_allclose(dn.logsigmoid(np.array([50.0, -50.0])), [0.0, -50.0], atol=1e-15)
    np.testing.assert_allclose(dn.logsigmoid(x) - dn.logsigmoid(-x), x, atol=1e-12)
