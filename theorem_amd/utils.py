"""Harness helpers with the behaviour of the reference's utils.py (:20-154):
seeding, the tolerance check used by every parity test, task.yml loading and
importing a kernel package by directory."""
from __future__ import annotations

import importlib
import random
import sys
from contextlib import contextmanager
from pathlib import Path
from typing import Any, Callable

import numpy as np
import torch


def set_seed(seed: int) -> None:
    """Seed Python, NumPy and torch (all devices)."""
    random.seed(seed)
    np.random.seed(seed)
    torch.manual_seed(seed)
    if torch.cuda.is_available():
        torch.cuda.manual_seed_all(seed)


def verbose_allclose(received, expected, rtol: float, atol: float, max_print: int = 5) -> list[str]:
    """Mismatch reasons (empty list = pass).  Containers are compared element-wise;
    a dtype difference is reported; NaN / Inf patterns must match; finite
    elements pass when |r - e| <= atol + rtol |e| (reference utils.py:30-83)."""
    if isinstance(received, (tuple, list)) or isinstance(expected, (tuple, list)):
        if type(received) is not type(expected) or len(received) != len(expected):
            return [f"container mismatch: received={type(received).__name__}, expected={type(expected).__name__}"]
        out: list[str] = []
        for i, (r, e) in enumerate(zip(received, expected)):
            out += [f"[{i}] {m}" for m in verbose_allclose(r, e, rtol, atol, max_print)]
        return out
    if not isinstance(received, torch.Tensor) or not isinstance(expected, torch.Tensor):
        return [f"type mismatch: received={type(received)}, expected={type(expected)}"]
    if received.shape != expected.shape:
        return [f"shape mismatch: received={tuple(received.shape)}, expected={tuple(expected.shape)}"]
    reasons: list[str] = []
    if received.dtype != expected.dtype:
        reasons.append(f"dtype mismatch: received={received.dtype}, expected={expected.dtype}")
    r = received.detach().float().cpu()
    e = expected.detach().float().cpu()
    if (torch.isnan(r) ^ torch.isnan(e)).any():
        reasons.append(f"NaN pattern mismatch in {int((torch.isnan(r) ^ torch.isnan(e)).sum())} elements")
    if (torch.isinf(r) ^ torch.isinf(e)).any():
        reasons.append(f"Inf pattern mismatch in {int((torch.isinf(r) ^ torch.isinf(e)).sum())} elements")
    fin = torch.isfinite(r) & torch.isfinite(e)
    diff = torch.where(fin, (r - e).abs(), torch.zeros_like(r))
    bad = fin & (diff > atol + rtol * e.abs())
    if bad.any():
        reasons.append(f"{int(bad.sum())} elements exceed tolerance (rtol={rtol}, atol={atol}); "
                       f"max|diff|={float(diff.max()):.3e}")
        for idx in torch.nonzero(bad)[:max_print]:
            t = tuple(int(i) for i in idx)
            reasons.append(f"  at {t}: received={float(r[t]):.6g}, expected={float(e[t]):.6g}")
    return reasons


def make_match_reference(ref_fn: Callable, rtol: float, atol: float):
    """A checker (data, output) -> (ok, message) against ref_fn(data)."""
    def check(data: Any, output) -> tuple[bool, str]:
        expected = ref_fn(*data) if isinstance(data, (tuple, list)) else ref_fn(data)
        reasons = verbose_allclose(output, expected, rtol=rtol, atol=atol)
        return not reasons, "; ".join(reasons)
    return check


@contextmanager
def DeterministicContext():
    """torch.use_deterministic_algorithms(True, warn_only=True) for the block.
    (The HIP kernels are deterministic on their own: no atomics, each output
    element written by one lane.)"""
    prev = torch.are_deterministic_algorithms_enabled()
    torch.use_deterministic_algorithms(True, warn_only=True)
    try:
        yield
    finally:
        torch.use_deterministic_algorithms(prev, warn_only=True)


def load_task(kernel_dir: Path) -> dict:
    import yaml

    with open(Path(kernel_dir) / "task.yml") as f:
        return yaml.safe_load(f)


def import_kernel(kernel_dir: Path) -> tuple[Callable, Callable]:
    """(custom_kernel, ref_kernel) of kernels/<name>/, imported as the package
    ``theorem_amd.kernels.<name>`` (reference utils.py:128-154 imports
    ``kernels.<name>`` from its project root)."""
    kernel_dir = Path(kernel_dir).resolve()
    if not (kernel_dir / "__init__.py").exists():
        raise FileNotFoundError(f"missing __init__.py at {kernel_dir}")
    pkg_root = kernel_dir.parent.parent  # the theorem_amd package directory
    repo_root = str(pkg_root.parent)
    if repo_root not in sys.path:
        sys.path.insert(0, repo_root)
    module = importlib.import_module(f"{pkg_root.name}.kernels.{kernel_dir.name}")
    custom = getattr(module, "custom_kernel", None)
    ref = getattr(module, "ref_kernel", None)
    if custom is None or ref is None:
        raise AttributeError(f"{kernel_dir} must export custom_kernel and ref_kernel")
    return custom, ref
