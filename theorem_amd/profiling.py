"""Helpers for the rocprofv3 counter summaries that bench.py reads.

``source_digest(unit)`` hashes a kernel's HIP source and every header it
includes (transitively, by ``#include "..."``), so a summary recorded with a
digest can be recognised as stale once the kernel's code has changed.

``traffic_summary(...)`` turns the counter CSVs of two ``rocprofv3 --pmc``
passes (FETCH_SIZE, then WRITE_SIZE) into HBM bytes per launch, scaled by the
calibration of a plain device copy of known size, and records the digest of
the kernel's sources beside them.

    python -m theorem_amd.profiling traffic OUT.json CALIB_FETCH_DIR CALIB_WRITE_DIR COPY_BYTES \\
        name=unit:symbol_prefix:algorithmic_bytes:FETCH_DIR:WRITE_DIR ...

``unit`` is a key of ``UNITS`` or the kernel's ``.hip`` file under csrc/.
"""
from __future__ import annotations

import csv
import glob
import hashlib
import json
import re
import sys
from pathlib import Path

CSRC = Path(__file__).resolve().parent / "csrc"
INCLUDE = CSRC.parent.parent / "include"

# bench.py kernel name -> the compilation unit its kernel lives in
UNITS = {
    "causal_conv1d": "causal_conv1d.hip",
    "recompute_w_u": "recompute_w_u.hip",
    "chunk_fwd_h": "chunk_fwd_h.hip",
    "chunk_fwd_o": "chunk_fwd_o.hip",
    "wy_build_A": "wy_build_A.hip",
    "chunk_gated_delta_fwd": "chunk_fwd_fused.hip",
    "chunk_gated_delta_fwd_a": "chunk_fwd_fused.hip",
    "wy_fwd": "wy_fwd.hip",
}

_INC = re.compile(r'^\s*#\s*include\s+"([^"]+)"', re.M)


def _sources(unit: str) -> list[Path]:
    if not (CSRC / unit).is_file():
        raise FileNotFoundError(f"no kernel source {CSRC / unit}")
    seen: dict[Path, None] = {}
    todo = [CSRC / unit]
    while todo:
        p = todo.pop()
        if p in seen or not p.exists():
            continue
        seen[p] = None
        for inc in _INC.findall(p.read_text()):
            todo.append((p.parent / inc).resolve())
    return sorted(seen)


def source_digest(unit: str) -> str:
    """sha256 (16 hex digits) over the unit's source and its included headers."""
    h = hashlib.sha256()
    for p in _sources(unit):
        h.update(p.name.encode())
        h.update(p.read_bytes())
    return h.hexdigest()[:16]


def _counter_kib(run_dir: str, counter: str, symbol_prefix: str) -> float:
    """Mean per-dispatch value of `counter` over the dispatches whose kernel name
    starts with `symbol_prefix` in a rocprofv3 counter_collection.csv."""
    f = glob.glob(str(Path(run_dir) / "**" / "*counter_collection.csv"), recursive=True)
    if not f:
        raise FileNotFoundError(f"no counter_collection.csv under {run_dir}")
    vals = [float(r["Counter_Value"]) for r in csv.DictReader(open(f[0]))
            if r["Counter_Name"] == counter and r["Kernel_Name"].startswith(symbol_prefix)]
    if not vals:
        raise ValueError(f"no {counter} dispatches of {symbol_prefix} in {f[0]}")
    return sum(vals) / len(vals)


# The runtime's device-to-device copy kernel (what `bench.py --copy-calib` runs
# for `Tensor.copy_`); the calibration averages only its dispatches, not the
# fill that initialises the source.
COPY_KERNEL = "__amd_rocclr_copyBuffer"


def traffic_summary(calib_fetch: str, calib_write: str, copy_bytes: int, targets: dict) -> dict:
    """targets: name -> (unit, symbol_prefix, algorithmic_bytes, fetch_dir, write_dir)."""
    cf = _counter_kib(calib_fetch, "FETCH_SIZE", COPY_KERNEL)
    cw = _counter_kib(calib_write, "WRITE_SIZE", COPY_KERNEL)
    ff, fw = copy_bytes / 1024 / cf, copy_bytes / 1024 / cw
    out = {"_calibration": {"copy_bytes": copy_bytes, "fetch_kib_per_copy": cf, "write_kib_per_copy": cw,
                            "fetch_factor": ff, "write_factor": fw}}
    for name, (unit, sym, alg, fdir, wdir) in targets.items():
        fk, wk = _counter_kib(fdir, "FETCH_SIZE", sym), _counter_kib(wdir, "WRITE_SIZE", sym)
        rd, wr = int(fk * 1024 * ff), int(wk * 1024 * fw)
        out[name] = {"kernel_symbol": sym, "source_digest": source_digest(unit), "fetch_kib_raw": fk,
                     "write_kib_raw": wk, "hbm_read_bytes": rd, "hbm_write_bytes": wr,
                     "hbm_bytes_per_launch": rd + wr, "algorithmic_bytes": alg,
                     "ratio": round((rd + wr) / alg, 4)}
    return out


def main(argv: list[str]) -> int:
    if len(argv) < 6 or argv[1] != "traffic":
        print(__doc__)
        return 2
    out, cfd, cwd, copy_bytes = argv[2], argv[3], argv[4], int(argv[5])
    targets = {}
    for spec in argv[6:]:
        name, rest = spec.split("=", 1)
        unit, sym, alg, fdir, wdir = rest.split(":")
        targets[name] = (UNITS.get(unit, unit), sym, int(alg), fdir, wdir)
    res = traffic_summary(cfd, cwd, copy_bytes, targets)
    Path(out).write_text(json.dumps(res, indent=1) + "\n")
    print(json.dumps({k: v.get("ratio") for k, v in res.items() if k != "_calibration"}))
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
