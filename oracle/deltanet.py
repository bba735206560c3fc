"""TEST INFRASTRUCTURE — NumPy oracles for the Gated DeltaNet chunk ops (see oracle/__init__.py).

All functions take and return NumPy arrays in the reference layout
(per-token tensors [B, T, H, D], gates [B, T, H], states [B, NT, H, K, V]) and
compute in ``dtype`` (float64 by default, so the oracle itself adds no
rounding error worth mentioning at the tolerances used).  Internally the
chunk axis is split out as [B, H, NT, BT, D] and every (b, head) pair is
processed at once with batched matmuls; the chunk loop of the state
recurrence is sequential, as in the reference.
"""
from __future__ import annotations

import numpy as np

BT = 64


def _chunks(x: np.ndarray, bt: int, dtype) -> np.ndarray:
    """[B, T, H, *D] -> [B, H, NT, bt, *D]."""
    B, T, H = x.shape[:3]
    assert T % bt == 0, f"T={T} must be a multiple of {bt}"
    y = x.astype(dtype, copy=False).reshape(B, T // bt, bt, H, *x.shape[3:])
    return np.moveaxis(y, 3, 1)


def _unchunk(y: np.ndarray) -> np.ndarray:
    """[B, H, NT, bt, *D] -> [B, T, H, *D]."""
    B, H, NT, bt = y.shape[:4]
    return np.moveaxis(y, 1, 3).reshape(B, NT * bt, H, *y.shape[4:])


def chunk_local_cumsum(a: np.ndarray, bt: int = BT) -> np.ndarray:
    """Per-chunk cumulative sum along T of a [B, T, H] gate increment
    (the construction of chunk_fwd_h/reference.py:39-45 and recompute_w_u/reference.py:104-106)."""
    B, T, H = a.shape
    return np.cumsum(a.reshape(B, T // bt, bt, H), axis=2).reshape(B, T, H)


def logsigmoid(x: np.ndarray) -> np.ndarray:
    """log(sigmoid(x)) = min(x, 0) - log1p(exp(-|x|)) (the logsigmoid gate of the
    gated delta rule; the reference's generators use plain negative increments)."""
    return np.minimum(x, 0.0) - np.log1p(np.exp(-np.abs(x)))


# --------------------------------------------------------------------------- chunk_fwd_h

def chunk_fwd_h_ref(k, v, g, bt: int = BT, dtype=np.float64) -> np.ndarray:
    """Reference form, chunk_fwd_h/reference.py:50-97.

    For each (b, head): state = 0; for each chunk c:
        diff = g_end - g_c;  state = state * exp(g_end) + k_c^T (v_c * exp(diff));  h[c] = state
    Returns h [B, NT, H, K, V].
    """
    kc, vc, gc = _chunks(k, bt, dtype), _chunks(v, bt, dtype), _chunks(g, bt, dtype)
    B, H, NT, _, K = kc.shape
    V = vc.shape[-1]
    state = np.zeros((B, H, K, V), dtype=dtype)
    h = np.zeros((B, NT, H, K, V), dtype=dtype)
    for c in range(NT):
        g_end = gc[:, :, c, -1]                                           # reference.py:86
        v_gated = vc[:, :, c] * np.exp(g_end[..., None] - gc[:, :, c])[..., None]   # :87-90
        state = state * np.exp(g_end)[..., None, None] + np.swapaxes(kc[:, :, c], -1, -2) @ v_gated  # :93
        h[:, c] = state                                                    # :95
    return h


def chunk_fwd_h_delta(k, w, u, g, h0=None, bt: int = BT, dtype=np.float64):
    """Delta-rule form (the chunk_fwd_h of BASELINE.json config 3; no counterpart
    in the reference, whose chunk_fwd_h is the form above).

    For each (b, head), S = h0 (or 0); for each chunk c:
        h[c] = S;  v_new_c = u_c - w_c S;  S = exp(g_last) S + (k_c * exp(g_last - g_c))^T v_new_c
    Returns (h [B, NT, H, K, V], v_new [B, T, H, V], final S [B, H, K, V]).
    """
    kc, wc, uc = _chunks(k, bt, dtype), _chunks(w, bt, dtype), _chunks(u, bt, dtype)
    gc = _chunks(g, bt, dtype) if g is not None else np.zeros(kc.shape[:4], dtype=dtype)
    B, H, NT, _, K = kc.shape
    V = uc.shape[-1]
    S = np.zeros((B, H, K, V), dtype=dtype) if h0 is None else h0.astype(dtype).copy()
    h = np.zeros((B, NT, H, K, V), dtype=dtype)
    vn = np.zeros_like(uc)
    for c in range(NT):
        h[:, c] = S
        vn[:, :, c] = uc[:, :, c] - wc[:, :, c] @ S
        g_last = gc[:, :, c, -1]
        kg = kc[:, :, c] * np.exp(g_last[..., None] - gc[:, :, c])[..., None]
        S = S * np.exp(g_last)[..., None, None] + np.swapaxes(kg, -1, -2) @ vn[:, :, c]
    return h, _unchunk(vn), S


# --------------------------------------------------------------------------- chunk_fwd_o

def chunk_fwd_o_ref(q, k, v, g, h, scale: float, bt: int = BT, dtype=np.float64) -> np.ndarray:
    """Factored form of chunk_fwd_o/reference.py:80-142:
        q_g = q e^{g}, v_g = v e^{-g};  qk = mask_incl(q_g k^T);  o = scale (qk v_g + q_g h[c])
    (mask keeps s <= t, diagonal included: reference.py:129-131).  Returns o [B, T, H, V]."""
    qc, kc, vc = _chunks(q, bt, dtype), _chunks(k, bt, dtype), _chunks(v, bt, dtype)
    gc = _chunks(g, bt, dtype)
    hc = np.moveaxis(h.astype(dtype, copy=False), 2, 1)                   # [B, H, NT, K, V]
    q_g = qc * np.exp(gc)[..., None]                                      # reference.py:116
    v_g = vc * np.exp(-gc)[..., None]                                     # :123
    qk = q_g @ np.swapaxes(kc, -1, -2)                                    # :126
    mask = np.tril(np.ones((bt, bt), dtype=bool))                         # :129-130
    qk = np.where(mask, qk, 0.0)                                          # :131
    o = scale * (qk @ v_g + q_g @ hc)                                     # :134-140
    return _unchunk(o)


def chunk_fwd_o_diff(q, k, v, g, h, scale: float, bt: int = BT, dtype=np.float64) -> np.ndarray:
    """The same output in gate-difference form (what the GPU kernel evaluates):
        o_i = scale ( sum_{j<=i} (q_i.k_j) e^{g_i-g_j} v_j + e^{g_i} q_i.h[c] )"""
    qc, kc, vc = _chunks(q, bt, dtype), _chunks(k, bt, dtype), _chunks(v, bt, dtype)
    gc = _chunks(g, bt, dtype) if g is not None else np.zeros(qc.shape[:4], dtype=dtype)
    hc = np.moveaxis(h.astype(dtype, copy=False), 2, 1)
    mask = np.tril(np.ones((bt, bt), dtype=bool))
    gate = np.exp(np.where(mask, gc[..., :, None] - gc[..., None, :], -np.inf))
    P = (qc @ np.swapaxes(kc, -1, -2)) * gate
    o = scale * (P @ vc + np.exp(gc)[..., None] * (qc @ hc))
    return _unchunk(o)


# --------------------------------------------------------------------------- recompute_w_u

def recompute_w_u_ref(k, v, beta, A, g, bt: int = BT, dtype=np.float64):
    """recompute_w_u/reference.py:118-149: per chunk, u = A_c (v * beta), w = A_c (k * beta e^{g}).
    A [B, T, H, bt] holds row r of A_c at t = c*bt + r (reference.py:88-90, 137).  Returns (w, u)."""
    kc, vc, bc = _chunks(k, bt, dtype), _chunks(v, bt, dtype), _chunks(beta, bt, dtype)
    gc = _chunks(g, bt, dtype) if g is not None else np.zeros(bc.shape, dtype=dtype)
    Ac = _chunks(A, bt, dtype)                                            # [B, H, NT, bt, bt]
    v_scaled = vc * bc[..., None]                                         # reference.py:140
    k_scaled = kc * (bc * np.exp(gc))[..., None]                          # :141
    return _unchunk(Ac @ k_scaled), _unchunk(Ac @ v_scaled)               # :143-144


def build_A(k, beta, g, sign: int = -1, bt: int = BT, dtype=np.float64) -> np.ndarray:
    """The WY matrix of recompute_w_u/reference.py:48-91:
        M = strict_lower( beta_i (k_i . k_j) e^{g_i - g_j} ),  A_c = (I - M)^{-1}   (sign = -1)
    sign = +1 gives (I + M)^{-1}, the gated-delta-rule form of BASELINE.json config 1.
    Solved per chunk with a dense LAPACK solve.  Returns A [B, T, H, bt]."""
    kc, bc = _chunks(k, bt, dtype), _chunks(beta, bt, dtype)
    gc = _chunks(g, bt, dtype) if g is not None else np.zeros(bc.shape, dtype=dtype)
    kkt = kc @ np.swapaxes(kc, -1, -2)
    M = kkt * bc[..., None] * np.exp(gc[..., :, None] - gc[..., None, :])
    M = np.tril(M, -1)
    eye = np.eye(bt, dtype=dtype)
    Ac = np.linalg.solve(eye + sign * M, np.broadcast_to(eye, M.shape))
    return _unchunk(Ac)


# --------------------------------------------------------------------------- full chain

def chunk_gated_delta_forward(q, k, v, beta, g, scale: float, h0=None, bt: int = BT,
                              dtype=np.float64):
    """Gated DeltaNet chunk forward composed from the ops above:
        A = (I + M)^{-1};  (w, u) = recompute_w_u;  (h, v_new, S) = chunk_fwd_h (delta form);
        o = chunk_fwd_o(q, k, v_new, g, h).
    ``g`` is the chunk-local cumulative log gate.  Returns (o, final S, intermediates dict)."""
    A = build_A(k, beta, g, sign=+1, bt=bt, dtype=dtype)
    w, u = recompute_w_u_ref(k, v, beta, A, g, bt=bt, dtype=dtype)
    h, v_new, S = chunk_fwd_h_delta(k, w, u, g, h0=h0, bt=bt, dtype=dtype)
    o = chunk_fwd_o_diff(q, k, v_new, g, h, scale, bt=bt, dtype=dtype)
    return o, S, {"A": A, "w": w, "u": u, "h": h, "v_new": v_new}


def gated_delta_rule_tokens(q, k, v, beta, a, scale: float, h0=None, dtype=np.float64):
    """Token-by-token gated delta rule (no chunking), the recurrence the chunked
    chain must reproduce.  ``a`` [B, T, H] is the per-token log decay (g is its
    chunk-local cumsum).  For each (b, head), with S [K, V]:
        S = e^{a_t} S;  S = S + beta_t k_t (v_t - S^T k_t)^T;  o_t = scale S^T q_t
    Returns (o [B, T, H, V], final S [B, H, K, V])."""
    B, T, H, K = k.shape
    V = v.shape[-1]
    q, k, v = q.astype(dtype), k.astype(dtype), v.astype(dtype)
    beta, a = beta.astype(dtype), a.astype(dtype)
    S = np.zeros((B, H, K, V), dtype=dtype) if h0 is None else h0.astype(dtype).copy()
    o = np.zeros((B, T, H, V), dtype=dtype)
    for t in range(T):
        S = S * np.exp(a[:, t])[..., None, None]
        kt, vt, qt = k[:, t], v[:, t], q[:, t]                            # [B, H, K] / [B, H, V]
        pred = np.einsum("bhkv,bhk->bhv", S, kt)
        S = S + np.einsum("bhk,bhv->bhkv", kt, beta[:, t][..., None] * (vt - pred))
        o[:, t] = scale * np.einsum("bhkv,bhk->bhv", S, qt)
    return o, S
