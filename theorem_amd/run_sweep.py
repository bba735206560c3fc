"""Multi-kernel sweep into one CSV, with the interface of the reference's
run_sweep.py (CSV schema :33-38, modes test/bench/both, one row per task.yml
shape, per-row failures in the ``error`` column without aborting the sweep).

    python -m theorem_amd.run_sweep [--kernels a,b] [--mode test|bench|both] [--out-dir DIR]

Writes DIR/sweep_<timestamp>.csv (default DIR: ./results) and prints a
markdown summary.  ``test`` rows run ref_kernel and custom_kernel on the
seeded task.yml test shapes and record correctness and max |diff|; ``bench``
rows time custom_kernel on the benchmark shapes (5 warm-up calls, then 50
calls each bracketed by a GPU event pair: min / p50 / mean in microseconds).
"""
from __future__ import annotations

import argparse
import csv
import datetime as _dt
import sys
import traceback
from pathlib import Path
from typing import Any

if __package__ in (None, ""):
    sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
    __package__ = "theorem_amd"

import torch  # noqa: E402

from .eval import _label, _load_inputs, _time_kernel  # noqa: E402
from .utils import DeterministicContext, import_kernel, load_task, set_seed, verbose_allclose  # noqa: E402

KERNELS_DIR = Path(__file__).resolve().parent / "kernels"
DEFAULT_KERNELS = ["causal_conv1d", "chunk_fwd_h", "chunk_fwd_o", "recompute_w_u"]
DEFAULT_SEED = 0

# Column order of the reference's sweep CSV.
CSV_COLUMNS = [
    "kernel", "shape", "mode",
    "B", "D_or_H", "S_or_T", "K", "V", "W",
    "min_us", "p50_us", "mean_us",
    "correct", "max_abs_diff", "error",
]

# Shape keys that fill each dimension column (first present wins).
_DIM_KEYS = {
    "B": ("B", "batch"),
    "D_or_H": ("D", "H", "n_heads", "dim"),
    "S_or_T": ("S", "T", "seqlen", "L"),
    "K": ("K", "chunk", "chunk_size"),
    "V": ("V", "vdim"),
    "W": ("W", "width", "kernel_size"),
}


def make_row(kernel: str, shape: dict, mode: str) -> dict:
    row: dict[str, Any] = {c: "" for c in CSV_COLUMNS}
    row.update(kernel=kernel, shape=_label(shape), mode=mode)
    for col, keys in _DIM_KEYS.items():
        row[col] = next((shape[k] for k in keys if k in shape), "")
    return row


def max_abs_diff(received, expected) -> float:
    """Largest finite |received - expected| over tensors or tuples of tensors; NaN if none."""
    pairs = list(zip(received, expected)) if isinstance(received, (tuple, list)) else [(received, expected)]
    best = float("nan")
    for r, e in pairs:
        if not (isinstance(r, torch.Tensor) and isinstance(e, torch.Tensor)) or r.shape != e.shape:
            return float("nan")
        rf, ef = r.detach().float().cpu(), e.detach().float().cpu()
        fin = torch.isfinite(rf) & torch.isfinite(ef)
        if fin.any():
            d = float((rf - ef).abs()[fin].max())
            best = d if best != best else max(best, d)
    return best


def sweep_kernel(kernel: str, mode: str, kernels_dir: Path = KERNELS_DIR) -> list[dict]:
    rows: list[dict] = []
    kdir = kernels_dir / kernel
    if not kdir.exists():
        return [{**make_row(kernel, {}, mode), "error": f"missing kernel dir: {kdir}"}]
    try:
        task = load_task(kdir)
        tols = task.get("tolerances", {}) or {}
        rtol, atol = float(tols.get("rtol", 1e-3)), float(tols.get("atol", 1e-3))
        custom_kernel, ref_kernel = import_kernel(kdir)
    except Exception as exc:  # noqa: BLE001
        return [{**make_row(kernel, {}, mode), "error": f"setup-failed: {type(exc).__name__}: {exc}"}]

    shapes = task.get("shapes", {}) or {}
    if mode in ("test", "both"):
        for shape in shapes.get("tests", []) or []:
            row = make_row(kernel, shape, "test")
            try:
                set_seed(int(shape.get("seed", DEFAULT_SEED)))
                with DeterministicContext():
                    data = _load_inputs(kdir, {k: v for k, v in shape.items() if k != "name"})
                    expected = ref_kernel(data)
                    received = custom_kernel(data)
                reasons = verbose_allclose(received, expected, rtol=rtol, atol=atol)
                row["correct"] = "false" if reasons else "true"
                row["max_abs_diff"] = f"{max_abs_diff(received, expected):.6g}"
                row["error"] = " | ".join(reasons[:3])
            except Exception as exc:  # noqa: BLE001
                row.update(correct="false", error=f"{type(exc).__name__}: {exc}")
            rows.append(row)
    if mode in ("bench", "both"):
        for shape in shapes.get("benchmarks", []) or []:
            row = make_row(kernel, shape, "bench")
            try:
                set_seed(int(shape.get("seed", DEFAULT_SEED)))
                data = _load_inputs(kdir, {k: v for k, v in shape.items() if k != "name"})
                mean, p50, mn, _ = _time_kernel(custom_kernel, data)
                row.update(min_us=f"{mn:.3f}", p50_us=f"{p50:.3f}", mean_us=f"{mean:.3f}")
            except Exception as exc:  # noqa: BLE001
                row["error"] = f"{type(exc).__name__}: {exc}"
            rows.append(row)
    return rows


def write_csv(rows: list[dict], out_dir: Path) -> Path:
    out_dir.mkdir(parents=True, exist_ok=True)
    path = out_dir / f"sweep_{_dt.datetime.now().strftime('%Y%m%d_%H%M%S')}.csv"
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=CSV_COLUMNS)
        w.writeheader()
        for row in rows:
            w.writerow({c: row.get(c, "") for c in CSV_COLUMNS})
    return path


def print_summary(rows: list[dict]) -> None:
    print("\n## Sweep summary\n")
    print("| kernel | shape | mode | min_us | p50_us | mean_us | correct | error |")
    print("|---|---|---|---:|---:|---:|---|---|")
    for r in rows:
        err = (r["error"] or "").replace("|", "\\|")[:60]
        print(f"| {r['kernel']} | {r['shape']} | {r['mode']} | {r['min_us'] or '-'} | {r['p50_us'] or '-'} | "
              f"{r['mean_us'] or '-'} | {r['correct'] or '-'} | {err} |")


def main(argv: list[str] | None = None) -> int:
    p = argparse.ArgumentParser(description="Sweep the MI355X kernels into a single CSV")
    p.add_argument("--kernels", default=",".join(DEFAULT_KERNELS), help="comma-separated kernel names")
    p.add_argument("--mode", choices=["test", "bench", "both"], default="both")
    p.add_argument("--out-dir", type=Path, default=Path("results"))
    args = p.parse_args(argv)
    kernels = [k.strip() for k in args.kernels.split(",") if k.strip()]
    print(f"PyTorch {torch.__version__} | ROCm/HIP {getattr(torch.version, 'hip', None)} | "
          f"GPU available: {torch.cuda.is_available()}")
    print(f"Sweeping kernels: {kernels} | mode: {args.mode}")
    rows: list[dict] = []
    for k in kernels:
        try:
            rows.extend(sweep_kernel(k, args.mode))
        except Exception as exc:  # noqa: BLE001 - keep the sweep alive
            traceback.print_exc()
            rows.append({**make_row(k, {}, args.mode), "error": f"sweep-aborted: {exc}"})
    path = write_csv(rows, args.out_dir)
    print(f"\nWrote {len(rows)} rows to {path}")
    print_summary(rows)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
