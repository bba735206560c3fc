"""Per-kernel correctness and latency driver, with the behaviour of the
reference's eval.py (:63-181):

    python -m theorem_amd.eval test|benchmark|both theorem_amd/kernels/<name>/

``test`` runs every task.yml test shape: seeded inputs from the package's
generate_input, ref_kernel vs custom_kernel, verbose_allclose at the task
tolerances.  ``benchmark`` times custom_kernel on the task.yml benchmark
shapes: 5 warm-up calls, then 50 calls each bracketed by a GPU event pair
(mean / p50 / min, host launch included, as the reference measures), plus
the device time per call of 200 back-to-back calls under one event pair.
"""
from __future__ import annotations

import argparse
import importlib
import sys
import traceback
from pathlib import Path

if __package__ in (None, ""):
    sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
    __package__ = "theorem_amd"

import torch  # noqa: E402

from .utils import DeterministicContext, import_kernel, load_task, set_seed, verbose_allclose  # noqa: E402

WARMUP_ITERS = 5
TIMED_ITERS = 50
BATCHED_ITERS = 200
DEFAULT_SEED = 0


def _print_header() -> None:
    print("=" * 72)
    print(f"PyTorch:      {torch.__version__}")
    print(f"ROCm/HIP:     {getattr(torch.version, 'hip', None) or 'n/a'}")
    from .kernels import _capi
    try:
        lib = _capi.load_library()
        print(f"Library:      {_capi.LIB_PATH} (ABI {lib.thm_abi_version()})")
    except RuntimeError as exc:
        print(f"Library:      NOT LOADED ({exc})")
    print(f"GPU:          {torch.cuda.get_device_name(0) if torch.cuda.is_available() else 'NOT AVAILABLE'}")
    print("=" * 72)


def _load_inputs(kernel_dir: Path, shape: dict):
    kernel_dir = Path(kernel_dir).resolve()
    mod = importlib.import_module(f"{kernel_dir.parent.parent.name}.kernels.{kernel_dir.name}.reference")
    gen = getattr(mod, "generate_input", None)
    if gen is None:
        raise AttributeError(f"{kernel_dir}/reference.py must export generate_input(**kwargs)")
    return gen(**shape)


def _label(shape: dict) -> str:
    return ", ".join(f"{k}={v}" for k, v in shape.items() if k != "name")


def run_tests(kernel_dir: Path) -> tuple[int, int]:
    task = load_task(kernel_dir)
    tests = task.get("shapes", {}).get("tests", []) or []
    tols = task.get("tolerances", {}) or {}
    rtol, atol = float(tols.get("rtol", 1e-3)), float(tols.get("atol", 1e-3))
    custom_kernel, ref_kernel = import_kernel(kernel_dir)
    passed = 0
    print(f"\n[test] {kernel_dir}  ({len(tests)} shapes; rtol={rtol}, atol={atol})")
    for shape in tests:
        label = _label(shape)
        try:
            set_seed(int(shape.get("seed", DEFAULT_SEED)))
            with DeterministicContext():
                data = _load_inputs(kernel_dir, {k: v for k, v in shape.items() if k != "name"})
                expected = ref_kernel(data)
                received = custom_kernel(data)
            reasons = verbose_allclose(received, expected, rtol=rtol, atol=atol)
            print(f"  {'PASS' if not reasons else 'FAIL'}  {label}")
            for r in reasons:
                print(f"        {r}")
            passed += not reasons
        except Exception as exc:  # noqa: BLE001 - report every failure mode per shape
            print(f"  ERROR {label}: {type(exc).__name__}: {exc}")
            traceback.print_exc(limit=2, file=sys.stdout)
    print(f"[test] {passed}/{len(tests)} passing")
    return passed, len(tests)


def _time_kernel(custom_kernel, data) -> tuple[float, float, float, float]:
    for _ in range(WARMUP_ITERS):
        custom_kernel(data)
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(TIMED_ITERS)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(TIMED_ITERS)]
    for i in range(TIMED_ITERS):
        starts[i].record()
        custom_kernel(data)
        ends[i].record()
    torch.cuda.synchronize()
    t = sorted(s.elapsed_time(e) * 1e3 for s, e in zip(starts, ends))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(BATCHED_ITERS):
        custom_kernel(data)
    e1.record()
    torch.cuda.synchronize()
    return sum(t) / len(t), t[len(t) // 2], t[0], e0.elapsed_time(e1) * 1e3 / BATCHED_ITERS


def run_benchmarks(kernel_dir: Path) -> None:
    task = load_task(kernel_dir)
    benches = task.get("shapes", {}).get("benchmarks", []) or []
    custom_kernel, _ = import_kernel(kernel_dir)
    print(f"\n[bench] {kernel_dir}  ({len(benches)} shapes; warmup={WARMUP_ITERS}, iters={TIMED_ITERS})")
    print(f"  {'shape':<48} {'mean_us':>9} {'p50_us':>9} {'min_us':>9} {'batched_us':>11}")
    for shape in benches:
        label = _label(shape)
        try:
            set_seed(int(shape.get("seed", DEFAULT_SEED)))
            data = _load_inputs(kernel_dir, {k: v for k, v in shape.items() if k != "name"})
            mean, p50, mn, batched = _time_kernel(custom_kernel, data)
            print(f"  {label:<48} {mean:>9.2f} {p50:>9.2f} {mn:>9.2f} {batched:>11.2f}")
        except Exception as exc:  # noqa: BLE001
            print(f"  {label:<48} ERROR: {type(exc).__name__}: {exc}")


def main(argv: list[str] | None = None) -> int:
    p = argparse.ArgumentParser(description="Theorem MI355X kernel eval harness")
    p.add_argument("mode", choices=["test", "benchmark", "both"])
    p.add_argument("kernel_dir", type=Path)
    args = p.parse_args(argv)
    _print_header()
    if not args.kernel_dir.exists():
        print(f"ERROR: kernel directory {args.kernel_dir} does not exist")
        return 2
    failed = False
    try:
        if args.mode in ("test", "both"):
            passed, total = run_tests(args.kernel_dir)
            failed = passed != total
        if args.mode in ("benchmark", "both"):
            run_benchmarks(args.kernel_dir)
    except Exception as exc:  # noqa: BLE001
        print(f"FATAL: {type(exc).__name__}: {exc}")
        traceback.print_exc()
        return 1
    return 1 if failed else 0


if __name__ == "__main__":
    raise SystemExit(main())
