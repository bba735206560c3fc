"""task.yml files carry the schema the reference's CI checks (.github/workflows/ci.yml:43-56)
and the reference's test shapes."""
from __future__ import annotations

from pathlib import Path

import pytest
import yaml

KDIR = Path(__file__).resolve().parent.parent / "theorem_amd" / "kernels"
NAMES = ["causal_conv1d", "chunk_fwd_h", "chunk_fwd_o", "recompute_w_u"]


@pytest.mark.parametrize("name", NAMES)
def test_schema(name):
    d = yaml.safe_load((KDIR / name / "task.yml").read_text())
    assert {"shapes", "tolerances"} <= d.keys()
    assert d["shapes"].get("tests") and d["shapes"].get("benchmarks")
    assert d["tolerances"]["rtol"] == 1e-2 and d["tolerances"]["atol"] == 1e-2
    for s in d["shapes"]["tests"] + d["shapes"]["benchmarks"]:
        assert "seed" in s


def test_packages_export_reference_interface():
    import importlib
    for n in NAMES:
        m = importlib.import_module(f"theorem_amd.kernels.{n}")
        assert callable(m.custom_kernel) and callable(m.ref_kernel) and callable(m.generate_input)
    wu = importlib.import_module("theorem_amd.kernels.recompute_w_u")
    for attr in ("generate_data", "Data", "BT", "SHAPE_CONFIGS", "SHAPE_LIST"):
        assert hasattr(wu, attr)
