"""The drop-in harness: eval.run_tests passes every task.yml test shape of
each kernel package (custom_kernel vs ref_kernel, the reference's own
tolerances and generators), and eval's timing path runs."""
from __future__ import annotations

from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

KDIR = Path(__file__).resolve().parent.parent / "theorem_amd" / "kernels"


@pytest.mark.parametrize("name", ["causal_conv1d", "chunk_fwd_h", "chunk_fwd_o", "recompute_w_u"])
def test_eval_run_tests(name, dev):
    from theorem_amd import eval as ev
    passed, total = ev.run_tests(KDIR / name)
    assert total > 0 and passed == total


def test_eval_timing_path(dev):
    from theorem_amd import eval as ev
    from theorem_amd.kernels import causal_conv1d
    data = causal_conv1d.generate_input(1, 64, 64, 4, 4242)
    mean, p50, mn, batched = ev._time_kernel(causal_conv1d.custom_kernel, data)
    assert 0 < mn <= p50 and batched > 0


def test_run_sweep_all_kernels(tmp_path):
    from theorem_amd import run_sweep
    rows = []
    for k in run_sweep.DEFAULT_KERNELS:
        rows += run_sweep.sweep_kernel(k, "test")
    assert rows and all(r["correct"] == "true" for r in rows), [r for r in rows if r["correct"] != "true"]
    bench = run_sweep.sweep_kernel("chunk_fwd_o", "bench")
    assert bench and all(float(r["min_us"]) > 0 and not r["error"] for r in bench)
    assert run_sweep.write_csv(rows + bench, tmp_path).exists()


def test_run_amd_smoke():
    from theorem_amd import run_amd
    assert run_amd.main([]) == 0
