"""Per-dispatch summary of a ``rocprofv3 --pmc`` run for one kernel.

Prints, for the dispatches of the kernel whose name contains ``--match``, the
median per-dispatch value of every collected counter (summed over the rows
rocprofv3 writes per dispatch), so a counter pass can be kept under
``profiles/`` as text next to the command that produced it.

Usage: python -m fa_amd.measure.counters <rocprofv3 output dir> --match hip_fa_fp32acc
"""

import argparse
import statistics

from fa_amd.measure.traffic import per_dispatch, pick


def summarize(folder, needle, counters):
    out = {}
    for name in counters:
        table = per_dispatch(folder, name)
        kernel = pick(table, needle)
        out[name] = (statistics.median(table[kernel]), len(table[kernel]), kernel)
    return out


def counter_names(folder):
    import csv
    import glob
    import os

    names = set()
    for path in glob.glob(os.path.join(folder, "**", "*counter_collection.csv"), recursive=True):
        with open(path, newline="", encoding="utf-8") as f:
            for row in csv.DictReader(f):
                names.add(row["Counter_Name"])
    return sorted(names)


def main(argv=None):
    p = argparse.ArgumentParser(description="per-dispatch PMC summary for one kernel")
    p.add_argument("folder")
    p.add_argument("--match", required=True)
    args = p.parse_args(argv)
    s = summarize(args.folder, args.match, counter_names(args.folder))
    kernel = next(iter(s.values()))[2] if s else "?"
    print(f"kernel: {kernel}")
    for name, (val, n, _) in s.items():
        print(f"{name:36s} {val:>22,.2f}   (median of {n} dispatches)")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
