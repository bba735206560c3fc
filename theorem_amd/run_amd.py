"""Quick smoke run of the four kernels, with the behaviour of the reference's
scripts/run_amd.py: print the environment, run ref_kernel and custom_kernel on
each kernel's smallest task.yml test shape, compare at rtol = atol = 1e-2, log
and continue past a failing kernel, print a PASS/FAIL summary.

    python -m theorem_amd.run_amd [--only causal_conv1d,chunk_fwd_h]

Exit status 0 when every selected kernel passes, 1 otherwise, 2 for an
unknown kernel name.
"""
from __future__ import annotations

import argparse
import importlib
import platform
import sys
import traceback
from pathlib import Path

if __package__ in (None, ""):
    sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
    __package__ = "theorem_amd"

ALL_KERNELS = ("causal_conv1d", "chunk_fwd_h", "chunk_fwd_o", "recompute_w_u")
TOL = {"rtol": 1e-2, "atol": 1e-2}
KERNELS_DIR = Path(__file__).resolve().parent / "kernels"


def smallest_shape(name: str) -> dict:
    """First test shape of the kernel's task.yml (its smallest case)."""
    from .utils import load_task

    shape = dict(load_task(KERNELS_DIR / name)["shapes"]["tests"][0])
    shape.pop("name", None)
    return shape


def print_env() -> None:
    print("=" * 60)
    print("Environment")
    print("=" * 60)
    print(f"Python : {platform.python_version()}  ({sys.executable})")
    try:
        import torch

        print(f"PyTorch: {torch.__version__}")
        print(f"HIP    : {getattr(torch.version, 'hip', None) or '(no HIP build)'}")
        print(f"GPU    : {torch.cuda.get_device_name(0) if torch.cuda.is_available() else '(no GPU detected)'}")
    except Exception as exc:  # noqa: BLE001
        print(f"PyTorch: import failed ({exc})")
    try:
        from .kernels import _capi

        lib = _capi.load_library()
        print(f"Library: {_capi.LIB_PATH} (ABI {lib.thm_abi_version()})")
    except Exception as exc:  # noqa: BLE001
        print(f"Library: not loaded ({exc})")
    print()


def _allclose(ref, got) -> bool:
    import torch

    if isinstance(ref, (tuple, list)):
        return isinstance(got, (tuple, list)) and len(ref) == len(got) and all(
            _allclose(r, g) for r, g in zip(ref, got))
    return ref.shape == got.shape and torch.allclose(got.float(), ref.float(), **TOL)


def run_one(name: str) -> bool:
    shape = smallest_shape(name)
    print(f"--- {name} (shape={shape}) ---")
    steps = (
        ("IMPORT/GEN", lambda st: st.update(
            mod=importlib.import_module(f"{__package__}.kernels.{name}"),
            data=importlib.import_module(f"{__package__}.kernels.{name}.reference").generate_input(**shape))),
        ("REF", lambda st: st.update(ref=st["mod"].ref_kernel(st["data"]))),
        ("CUSTOM", lambda st: st.update(got=st["mod"].custom_kernel(st["data"]))),
        ("COMPARE", lambda st: st.update(ok=_allclose(st["ref"], st["got"]))),
    )
    state: dict = {}
    for what, step in steps:
        try:
            step(state)
        except Exception as exc:  # noqa: BLE001 - log and continue with the next kernel
            print(f"  {what} FAIL: {exc}")
            traceback.print_exc(limit=2)
            return False
    ok = bool(state["ok"])
    print(f"  {'PASS' if ok else 'FAIL'}  (rtol={TOL['rtol']}, atol={TOL['atol']})")
    return ok


def main(argv: list[str] | None = None) -> int:
    p = argparse.ArgumentParser()
    p.add_argument("--only", default="", help=f"comma-separated subset of {','.join(ALL_KERNELS)}")
    args = p.parse_args(argv)
    selected = [s.strip() for s in args.only.split(",") if s.strip()] or list(ALL_KERNELS)
    bad = [s for s in selected if s not in ALL_KERNELS]
    if bad:
        print(f"ERROR: unknown kernel(s): {bad}; valid: {ALL_KERNELS}")
        return 2
    print_env()
    results = {name: run_one(name) for name in selected}
    print()
    print("=" * 60)
    print("Summary")
    print("=" * 60)
    for name, ok in results.items():
        print(f"  {name:18s}  {'PASS' if ok else 'FAIL'}")
    return 0 if all(results.values()) else 1


if __name__ == "__main__":
    raise SystemExit(main())
