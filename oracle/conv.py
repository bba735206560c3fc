"""TEST INFRASTRUCTURE — causal conv oracles (see oracle/__init__.py)."""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
_SO = _DIR / "_build" / "liboracle.so"
_lib = None


def build() -> Path:
    """Compile conv1d.c with the committed Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", str(_DIR)], check=True)
    return _SO


def _load():
    global _lib
    if _lib is None:
        if not _SO.exists():
            build()
        lib = ctypes.CDLL(str(_SO))
        f = lib.oracle_causal_conv1d_f32
        f.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int64] * 3 + [ctypes.c_int32]
        f.restype = None
        _lib = lib
    return _lib


def causal_conv1d_c(x: np.ndarray, weight: np.ndarray, bias: np.ndarray | None) -> np.ndarray:
    """C restatement (conv1d.c) of scripts/cpu_reference.py:40-63; fp32, single thread."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    weight = np.ascontiguousarray(weight, dtype=np.float32)
    B, D, S = x.shape
    W = weight.shape[1]
    out = np.empty_like(x)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    _load().oracle_causal_conv1d_f32(
        x.ctypes.data, weight.ctypes.data, None if b is None else b.ctypes.data, out.ctypes.data,
        B, D, S, W)
    return out


def causal_conv1d_numpy(x: np.ndarray, weight: np.ndarray, bias: np.ndarray | None,
                        dtype=np.float32) -> np.ndarray:
    """NumPy restatement of scripts/cpu_reference.py:40-63 (pad, out = bias, W tap passes)."""
    B, D, S = x.shape
    Dw, W = weight.shape
    assert D == Dw
    x = x.astype(dtype, copy=False)
    weight = weight.astype(dtype, copy=False)
    xp = np.pad(x, ((0, 0), (0, 0), (W - 1, 0)))                    # cpu_reference.py:54
    if bias is None:
        out = np.zeros((B, D, S), dtype=dtype)
    else:
        out = np.broadcast_to(bias.astype(dtype)[None, :, None], (B, D, S)).copy()  # :56
    for k in range(W):                                               # :58-62
        out += weight[None, :, k, None] * xp[:, :, k:k + S]
    return out


def causal_conv1d_bruteforce(x: np.ndarray, weight: np.ndarray, bias: np.ndarray | None) -> np.ndarray:
    """Direct double loop of out[b,d,t] = bias[d] + sum_k w[d,k] x[b,d,t-W+1+k] (float64)."""
    B, D, S = x.shape
    W = weight.shape[1]
    out = np.zeros((B, D, S), dtype=np.float64)
    for b in range(B):
        for d in range(D):
            for t in range(S):
                acc = 0.0 if bias is None else float(bias[d])
                for k in range(W):
                    s = t - W + 1 + k
                    if s >= 0:
                        acc += float(weight[d, k]) * float(x[b, d, s])
                out[b, d, t] = acc
    return out


def silu(x: np.ndarray) -> np.ndarray:
    return x / (1.0 + np.exp(-x))


def causal_conv1d_update_ref(x: np.ndarray, state: np.ndarray, weight: np.ndarray, bias: np.ndarray | None,
                             dtype=np.float64):
    """Decode step with a rolling state, restated from the conv's definition
    (scripts/cpu_reference.py:40-63 applied to the window state ++ x):
        window = state ++ x (along time),  out[t] = bias + sum_k w[k] window[L_s - W + 1 + t + k],
        new state = the last L_s samples of window.
    x [B, D, L], state [B, D, L_s].  Returns (out [B, D, L], new state)."""
    B, D, L = x.shape
    Ls = state.shape[2]
    W = weight.shape[1]
    win = np.concatenate([state.astype(dtype), x.astype(dtype)], axis=2)
    out = np.zeros((B, D, L), dtype=dtype) + (0 if bias is None else bias.astype(dtype)[None, :, None])
    for k in range(W):
        out += weight.astype(dtype)[None, :, k, None] * win[:, :, Ls - W + 1 + k:Ls - W + 1 + k + L]
    return out, win[:, :, L:]
