"""HIP kernels vs PyTorch eager vs torch.compile on the task.yml benchmark
shapes, with the behaviour of the reference's benchmarks/pytorch_baseline.py
(:72-468): 5 warm-up calls, then the minimum over 50 calls, each bracketed by
a GPU event pair and a synchronize; per-cell failures become NaN.

    python -m theorem_amd.benchmarks.pytorch_baseline [--kernels a,b] [--csv out.csv] [--no-compile]

The eager baselines are vectorised PyTorch forms of each op (only the state
recurrence keeps a Python loop over chunks).
"""
from __future__ import annotations

import argparse
import csv
import sys
import traceback
from pathlib import Path
from typing import Any, Callable, Dict, List

import torch
import torch.nn.functional as F
import yaml

PKG = Path(__file__).resolve().parent.parent
if str(PKG.parent) not in sys.path:
    sys.path.insert(0, str(PKG.parent))

WARMUP_ITERS = 5
TIMED_ITERS = 50


def _time_callable(fn: Callable[[], Any]) -> float:
    for _ in range(WARMUP_ITERS):
        fn()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(TIMED_ITERS):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        torch.cuda.synchronize()
        best = min(best, s.elapsed_time(e))
    return best * 1e3


def _safe_time(label: str, shape: dict, fn) -> float:
    try:
        return _time_callable(fn)
    except Exception as exc:  # noqa: BLE001 - a failing cell becomes NaN
        print(f"  [warn] {label} failed on {shape}: {type(exc).__name__}: {exc}", file=sys.stderr)
        traceback.print_exc(file=sys.stderr)
        return float("nan")


# ----------------------------------------------------------------- eager baselines

def conv_eager(x, w, b):
    return F.conv1d(F.pad(x, (w.shape[1] - 1, 0)), w.unsqueeze(1), bias=b, groups=x.shape[1])


def h_eager(k, v, g, BT=64):
    B, T, H, K = k.shape
    V = v.shape[-1]
    NT = T // BT
    kc, vc, gc = k.view(B, NT, BT, H, K), v.view(B, NT, BT, H, V), g.view(B, NT, BT, H)
    out = torch.empty(B, NT, H, K, V, device=k.device)
    S = torch.zeros(B, H, K, V, device=k.device)
    for c in range(NT):
        ge = gc[:, c, -1]
        vg = vc[:, c] * torch.exp(ge.unsqueeze(1) - gc[:, c]).unsqueeze(-1)
        S = S * torch.exp(ge)[..., None, None] + kc[:, c].permute(0, 2, 3, 1).contiguous() @ vg.permute(0, 2, 1, 3).contiguous()
        out[:, c] = S
    return out


def o_eager(q, k, v, g, h, scale, BT=64):
    B, T, H, K = q.shape
    V = v.shape[-1]
    NT = T // BT
    qc = q.view(B, NT, BT, H, K).permute(0, 1, 3, 2, 4)
    kc = k.view(B, NT, BT, H, K).permute(0, 1, 3, 2, 4)
    vc = v.view(B, NT, BT, H, V).permute(0, 1, 3, 2, 4)
    gc = g.view(B, NT, BT, H).permute(0, 1, 3, 2)
    qg = qc * torch.exp(gc).unsqueeze(-1)
    vg = (vc * torch.exp(-gc).unsqueeze(-1)).contiguous()
    qk = torch.tril(qg @ kc.transpose(-1, -2).contiguous())
    o = scale * (qk @ vg + qg @ h)
    return o.permute(0, 1, 3, 2, 4).reshape(B, T, H, V)


def wu_eager(k, v, beta, A, g, BT=64):
    B, T, H, K = k.shape
    V = v.shape[-1]
    NT = T // BT
    kc = k.view(B, NT, BT, H, K).permute(0, 1, 3, 2, 4)
    vc = v.view(B, NT, BT, H, V).permute(0, 1, 3, 2, 4)
    bc = beta.view(B, NT, BT, H).permute(0, 1, 3, 2)
    gc = g.view(B, NT, BT, H).permute(0, 1, 3, 2)
    Ac = A.view(B, NT, BT, H, BT).permute(0, 1, 3, 2, 4)
    u = Ac @ (vc * bc.unsqueeze(-1)).contiguous()
    w = Ac @ (kc * (bc * torch.exp(gc)).unsqueeze(-1)).contiguous()
    return (w.permute(0, 1, 3, 2, 4).reshape(B, T, H, K), u.permute(0, 1, 3, 2, 4).reshape(B, T, H, V))


# ----------------------------------------------------------------- stagers

def _stage(kname: str, shape: dict, compile_: bool):
    import importlib
    mod = importlib.import_module(f"theorem_amd.kernels.{kname}")
    args = {k: shape[k] for k in shape if k != "seed"}
    data = mod.generate_input(**args, seed=shape["seed"])
    if kname == "causal_conv1d":
        fn, eager_args = conv_eager, data
    elif kname == "chunk_fwd_h":
        fn, eager_args = h_eager, (data["k"], data["v"], data["g"])
    elif kname == "chunk_fwd_o":
        fn, eager_args = o_eager, (data["q"], data["k"], data["v"], data["g"], data["h"], data["scale"])
    else:
        fn, eager_args = wu_eager, (data.k, data.v, data.beta, data.A, data.g)
    compiled = torch.compile(fn, mode="max-autotune-no-cudagraphs") if compile_ else None
    return (lambda: mod.custom_kernel(data), lambda: fn(*eager_args),
            (lambda: compiled(*eager_args)) if compiled else None)


KERNELS = ["causal_conv1d", "chunk_fwd_h", "chunk_fwd_o", "recompute_w_u"]


def main(argv: List[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--kernels", default=",".join(KERNELS))
    ap.add_argument("--csv", default="gpurun_out/baseline_compare.csv")
    ap.add_argument("--no-compile", action="store_true", help="skip the torch.compile column")
    ap.add_argument("--max-shapes", type=int, default=0, help="only the first N benchmark shapes per kernel")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("error: no GPU device visible", file=sys.stderr)
        return 2
    rows: List[Dict[str, Any]] = []
    for kname in [s.strip() for s in args.kernels.split(",") if s.strip()]:
        shapes = yaml.safe_load((PKG / "kernels" / kname / "task.yml").read_text())["shapes"]["benchmarks"]
        if args.max_shapes:
            shapes = shapes[:args.max_shapes]
        print(f"\n=== {kname} ===")
        for shape in shapes:
            label = ",".join(f"{k}={v}" for k, v in shape.items() if k != "seed")
            try:
                run_hip, run_eager, run_comp = _stage(kname, shape, not args.no_compile)
            except Exception as exc:  # noqa: BLE001
                print(f"  [error] staging {label}: {exc}", file=sys.stderr)
                continue
            t = _safe_time("hip", shape, run_hip)
            e = _safe_time("eager", shape, run_eager)
            c = _safe_time("compiled", shape, run_comp) if run_comp else float("nan")
            rows.append({"kernel": kname, "shape": label, "hip_min_us": t, "eager_min_us": e, "compiled_min_us": c,
                         "hip_speedup_vs_eager": e / t if t == t and e == e else float("nan")})
            print(f"  {label}: hip {t:.2f} us  eager {e:.2f} us  compiled {c:.2f} us")
            torch.cuda.empty_cache()
    out = Path(args.csv)
    out.parent.mkdir(parents=True, exist_ok=True)
    with out.open("w", newline="") as fh:
        wr = csv.DictWriter(fh, fieldnames=list(rows[0].keys()) if rows else ["kernel"])
        wr.writeheader()
        wr.writerows(rows)
    print(f"\nwrote {out}")
    print("\n| kernel | shape | hip_min_us | eager_min_us | compiled_min_us | speedup vs eager |")
    print("| --- | --- | ---: | ---: | ---: | ---: |")
    for r in rows:
        print(f"| {r['kernel']} | {r['shape']} | {r['hip_min_us']:.2f} | {r['eager_min_us']:.2f} | "
              f"{r['compiled_min_us']:.2f} | {r['hip_speedup_vs_eager']:.2f}x |")
    return 0


if __name__ == "__main__":
    sys.exit(main())
