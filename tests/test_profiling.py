"""The counter-summary plumbing behind bench.py's ``roofline.traffic`` (CPU).

theorem_amd/profiling.py turns two rocprofv3 counter passes (FETCH_SIZE, then
WRITE_SIZE) into HBM bytes per launch, scaled by a calibration copy, and
stamps each entry with a digest of the kernel's sources; bench.py reports the
figure only while that digest matches the sources it runs.  These tests
check the digest's coverage (a change to any transitively included header
makes it stale, an unrelated file does not), the calibrated arithmetic on
synthetic counter CSVs, and bench.py's stale / missing handling.
"""
from __future__ import annotations

import csv
import importlib.util
import json
import shutil
from pathlib import Path

import pytest

from theorem_amd import profiling

ROOT = Path(__file__).resolve().parent.parent


def test_every_unit_digest_covers_its_headers():
    for name, unit in profiling.UNITS.items():
        srcs = {p.name for p in profiling._sources(unit)}
        assert unit in srcs, name
    fused = {p.name for p in profiling._sources("chunk_fwd_fused.hip")}
    # direct and transitive includes (pipe_cfg.h and vmem.h come in through
    # the unit, common.h through them)
    assert {"h_layout.h", "pipe_cfg.h", "vmem.h", "mfma.h", "common.h"} <= fused


def test_digest_changes_with_a_transitive_header_only(tmp_path, monkeypatch):
    csrc = tmp_path / "csrc"
    shutil.copytree(profiling.CSRC, csrc, ignore=shutil.ignore_patterns("*.o", "*.so", "host"))
    monkeypatch.setattr(profiling, "CSRC", csrc)
    d0 = profiling.source_digest("chunk_fwd_o.hip")
    assert d0 == profiling.source_digest("chunk_fwd_o.hip")
    # a file the unit does not include: digest unchanged
    (csrc / "wy_blocks.h").write_text((csrc / "wy_blocks.h").read_text() + "\n// edit\n")
    assert "wy_blocks.h" not in {p.name for p in profiling._sources("chunk_fwd_o.hip")}
    assert profiling.source_digest("chunk_fwd_o.hip") == d0
    # a header reached only through another header: digest changes
    (csrc / "common.h").write_text((csrc / "common.h").read_text() + "\n// edit\n")
    assert profiling.source_digest("chunk_fwd_o.hip") != d0


def test_unknown_unit_raises_and_cli_takes_units_keys(tmp_path):
    # A unit name that is no source file must not hash to the empty digest
    # (which would mark every summary built from it as matching nothing).
    with pytest.raises(FileNotFoundError):
        profiling.source_digest("chunk_fwd_h")
    calib, kern = tmp_path / "calib", tmp_path / "kern"
    _counter_csv(calib, [(profiling.COPY_KERNEL, "FETCH_SIZE", 512.0), (profiling.COPY_KERNEL, "WRITE_SIZE", 1024.0)])
    _counter_csv(kern, [("_ZN3thm6kernelEv", "FETCH_SIZE", 8.0), ("_ZN3thm6kernelEv", "WRITE_SIZE", 4.0)])
    out = tmp_path / "t.json"
    spec = f"chunk_fwd_h=chunk_fwd_h:_ZN3thm6kernel:24576:{kern}:{kern}"
    assert profiling.main(["profiling", "traffic", str(out), str(calib), str(calib), "1048576", spec]) == 0
    rec = json.loads(out.read_text())["chunk_fwd_h"]
    assert rec["source_digest"] == profiling.source_digest(profiling.UNITS["chunk_fwd_h"])
    assert rec["hbm_read_bytes"] == 8 * 1024 * 2 and rec["hbm_write_bytes"] == 4 * 1024


def _counter_csv(path: Path, rows):
    path.mkdir(parents=True, exist_ok=True)
    with open(path / "run_counter_collection.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for i, (kernel, counter, value) in enumerate(rows):
            w.writerow({"Dispatch_Id": i, "Kernel_Name": kernel, "Counter_Name": counter, "Counter_Value": value})


def test_traffic_summary_calibrates_and_averages_matching_dispatches(tmp_path):
    copy_bytes = 1 << 30
    copy_k = profiling.COPY_KERNEL + "(void*)"
    # FETCH_SIZE of the copy reads half the true bytes, WRITE_SIZE all of them;
    # the fill kernel of the calibration run is not averaged.
    _counter_csv(tmp_path / "cf", [(copy_k, "FETCH_SIZE", copy_bytes / 1024 / 2),
                                   ("fill_kernel", "FETCH_SIZE", 1.0)])
    _counter_csv(tmp_path / "cw", [(copy_k, "WRITE_SIZE", copy_bytes / 1024),
                                   (copy_k, "WRITE_SIZE", copy_bytes / 1024)])
    sym = "_ZN3thm12_GLOBAL__N_123chunk_fwd_o_pipe_kernel"
    _counter_csv(tmp_path / "f", [(sym + "ILi128E", "FETCH_SIZE", 900.0), (sym + "ILi128E", "FETCH_SIZE", 1100.0),
                                  ("other_kernel", "FETCH_SIZE", 1e9)])
    _counter_csv(tmp_path / "w", [(sym + "ILi128E", "WRITE_SIZE", 500.0)])
    res = profiling.traffic_summary(str(tmp_path / "cf"), str(tmp_path / "cw"), copy_bytes,
                                    {"chunk_fwd_o": ("chunk_fwd_o.hip", sym, 3_000_000,
                                                     str(tmp_path / "f"), str(tmp_path / "w"))})
    cal = res["_calibration"]
    assert cal["fetch_factor"] == pytest.approx(2.0) and cal["write_factor"] == pytest.approx(1.0)
    e = res["chunk_fwd_o"]
    assert e["fetch_kib_raw"] == pytest.approx(1000.0)  # mean of the two matching dispatches
    assert e["hbm_read_bytes"] == 1000 * 1024 * 2 and e["hbm_write_bytes"] == 500 * 1024
    assert e["hbm_bytes_per_launch"] == 1000 * 1024 * 2 + 500 * 1024
    assert e["ratio"] == pytest.approx(round((1000 * 1024 * 2 + 500 * 1024) / 3_000_000, 4))
    assert e["source_digest"] == profiling.source_digest("chunk_fwd_o.hip")
    with pytest.raises(ValueError):
        profiling.traffic_summary(str(tmp_path / "cf"), str(tmp_path / "cw"), copy_bytes,
                                  {"x": ("chunk_fwd_o.hip", "no_such_kernel", 1, str(tmp_path / "f"),
                                         str(tmp_path / "w"))})


def _bench_module():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_bench_reports_traffic_only_for_current_sources(tmp_path, monkeypatch):
    bench = _bench_module()
    monkeypatch.setattr(bench, "ROOT", tmp_path)
    (tmp_path / "profiles").mkdir()
    f = tmp_path / "profiles" / "traffic_cfg4.json"
    assert bench.measured_traffic("chunk_fwd_o")[0] is None  # no summary
    rec = {"source_digest": profiling.source_digest("chunk_fwd_o.hip"), "hbm_bytes_per_launch": 123,
           "ratio": 1.5, "algorithmic_bytes": 82}
    f.write_text(json.dumps({"chunk_fwd_o": rec}))
    assert bench.measured_traffic("chunk_fwd_o")[0] == 123
    assert bench.measured_traffic("chunk_fwd_h") == (None, "kernel not in the counter summary")
    f.write_text(json.dumps({"chunk_fwd_o": dict(rec, source_digest="0" * 16)}))
    by, note = bench.measured_traffic("chunk_fwd_o")
    assert by is None and note.startswith("stale")
