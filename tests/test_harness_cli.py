"""CPU checks of the sweep / smoke-run harness: the CSV schema is the
reference's (run_sweep.py:33-38), rows take their dimension columns from the
task.yml shape keys, and bad arguments are rejected before any GPU work."""
from __future__ import annotations

import csv

from theorem_amd import run_amd, run_sweep


def test_csv_schema_is_the_references():
    assert run_sweep.CSV_COLUMNS == [
        "kernel", "shape", "mode", "B", "D_or_H", "S_or_T", "K", "V", "W",
        "min_us", "p50_us", "mean_us", "correct", "max_abs_diff", "error"]


def test_rows_and_csv(tmp_path):
    conv = run_sweep.make_row("causal_conv1d", {"B": 1, "D": 64, "S": 128, "W": 4, "seed": 3}, "test")
    assert (conv["B"], conv["D_or_H"], conv["S_or_T"], conv["W"], conv["K"]) == (1, 64, 128, 4, "")
    h = run_sweep.make_row("chunk_fwd_h", {"B": 2, "T": 256, "H": 3, "K": 64, "V": 128, "seed": 1}, "bench")
    assert (h["D_or_H"], h["S_or_T"], h["K"], h["V"], h["mode"]) == (3, 256, 64, 128, "bench")
    assert h["shape"] == "B=2, T=256, H=3, K=64, V=128, seed=1"
    path = run_sweep.write_csv([conv, h], tmp_path)
    with open(path) as f:
        got = list(csv.DictReader(f))
    assert [r["kernel"] for r in got] == ["causal_conv1d", "chunk_fwd_h"] and list(got[0]) == run_sweep.CSV_COLUMNS


def test_missing_kernel_is_a_row_not_a_crash(tmp_path):
    rows = run_sweep.sweep_kernel("no_such_kernel", "test")
    assert len(rows) == 1 and rows[0]["error"].startswith("missing kernel dir")


def test_run_amd_rejects_unknown_kernel_and_knows_smallest_shapes():
    assert run_amd.main(["--only", "bogus"]) == 2
    assert run_amd.smallest_shape("causal_conv1d") == {"B": 1, "D": 64, "S": 64, "W": 4, "seed": 4242}
    assert run_amd.smallest_shape("recompute_w_u") == {"B": 1, "T": 64, "H": 2, "K": 64, "V": 64, "seed": 4242}
