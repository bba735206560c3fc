"""Table of lds_bank_probe's measured LDS bank conflicts beside the model's verdict.

Usage: python tests/csrc/lds_bank_summary.py PROBE_STDOUT COUNTER_CSV

PROBE_STDOUT holds the probe's lines (launch index, pattern, model slowdown);
COUNTER_CSV is rocprofv3's counter_collection.csv of the same run with
SQ_LDS_BANK_CONFLICT, SQ_LDS_IDX_ACTIVE and SQ_INSTS_LDS.  Prints a markdown
table: conflict cycles and active cycles per LDS instruction, and whether the
model (tests/csrc/lds_banks.h) agrees: "yes" when it calls a pattern
conflict-free exactly when the counter shows no conflict cycles,
"conservative" when it reports a conflict the counter does not show, "NO"
when it misses one (exit status 1).
"""
import collections
import csv
import sys


def main(probe_out: str, counters: str) -> int:
    pats = [line.rstrip("\n").split("\t") for line in open(probe_out) if line.count("\t") == 2]
    by_dispatch = collections.defaultdict(dict)
    for r in csv.DictReader(open(counters)):
        if "lds_probe" in r["Kernel_Name"]:
            by_dispatch[int(r["Dispatch_Id"])][r["Counter_Name"]] = float(r["Counter_Value"])
    rows = [by_dispatch[k] for k in sorted(by_dispatch)]
    if len(rows) != len(pats):
        print(f"{len(pats)} patterns but {len(rows)} probe dispatches", file=sys.stderr)
        return 1
    print("| pattern | conflict cycles / instr | active cycles / instr | model | agrees |")
    print("|---|---:|---:|---|---|")
    bad = cons = 0
    for (idx, name, ways), c in zip(pats, rows):
        n = c["SQ_INSTS_LDS"]
        conf, act = c["SQ_LDS_BANK_CONFLICT"] / n, c["SQ_LDS_IDX_ACTIVE"] / n
        model = "conflict-free" if ways == "1" else f"{ways}-way"
        if (ways == "1") == (conf == 0):
            verdict = "yes"
        elif conf == 0:
            verdict = "conservative"  # the model reports a conflict the counter does not show
            cons += 1
        else:
            verdict = "NO"  # a conflict the model misses
            bad += 1
        print(f"| {name} | {conf:.2f} | {act:.2f} | {model} | {verdict} |")
    print(f"\n{len(pats) - bad - cons} of {len(pats)} patterns agree with the model, {cons} conservatively "
          f"(reported as a conflict, measured free), {bad} missed.")
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1], sys.argv[2]))
