"""Per-kernel duration statistics of a ``rocprofv3 --kernel-trace`` run.

Reads the run's SQLite output (``*_results.db``, the default rocpd format:
view ``kernels`` with ``name`` and ``duration`` in ns) or, for runs made with
``--output-format csv``, ``*_kernel_stats.csv``, and prints one line per
kernel: calls, average/min/max duration in ns and share of the total. The
text is what ``profiles/`` keeps for a workload.

Usage: python -m fa_amd.measure.kernel_stats <rocprofv3 output dir> [--flops F --match NAME] [--skip N]
``--flops`` adds the achieved TFLOP/s of the kernel whose name contains
``--match`` (average duration). ``--skip N`` drops the first N dispatches of
every kernel (in launch order), so that a profile of ``bench.py`` averages its
timed steps only, not its warmup steps.
"""

import argparse
import csv
import glob
import os
import sqlite3
import statistics


def from_db(path):
    """{kernel name: [duration ns, ...]} in launch order (by start time when recorded)."""
    con = sqlite3.connect(path)
    try:
        cols = {row[1] for row in con.execute("PRAGMA table_info(kernels)")}
        order = "start" if "start" in cols else "rowid"
        rows = con.execute(f"SELECT name, duration FROM kernels ORDER BY {order}").fetchall()
    finally:
        con.close()
    out = {}
    for name, dur in rows:
        out.setdefault(name, []).append(float(dur))
    return out


def collect(folder):
    dbs = glob.glob(os.path.join(folder, "**", "*_results.db"), recursive=True)
    if dbs:
        merged = {}
        for db in dbs:
            for k, v in from_db(db).items():
                merged.setdefault(k, []).extend(v)
        return merged
    traces = glob.glob(os.path.join(folder, "**", "*_kernel_trace.csv"), recursive=True)
    timed = {}
    for path in traces:
        with open(path, newline="", encoding="utf-8") as f:
            for row in csv.DictReader(f):
                start, end = float(row["Start_Timestamp"]), float(row["End_Timestamp"])
                timed.setdefault(row["Kernel_Name"], []).append((start, end - start))
    if not timed:
        raise FileNotFoundError(f"no rocprofv3 kernel trace under {folder}")
    return {name: [d for _, d in sorted(v)] for name, v in timed.items()}


def skip_first(stats, n):
    """``stats`` without the first ``n`` dispatches of every kernel (launch order).

    A kernel with no more than ``n`` dispatches keeps its last one, so every
    kernel of the run still has a line.
    """
    if n <= 0:
        return dict(stats)
    return {name: (durs[n:] if len(durs) > n else durs[-1:]) for name, durs in stats.items()}


def short(name, width=72):
    return name if len(name) <= width else name[: width - 3] + "..."


def render(stats, flops=None, match=None):
    total = sum(sum(v) for v in stats.values())
    lines = [f"{'Name':<74} {'Calls':>5} {'AverageNs':>13} {'MinNs':>13} {'MaxNs':>13} {'Pct':>7}"]
    for name, durs in sorted(stats.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"{short(name):<74} {len(durs):>5} {statistics.mean(durs):>13,.0f} "
                     f"{min(durs):>13,.0f} {max(durs):>13,.0f} {100 * sum(durs) / total:>7.3f}")
    if flops and match:
        hits = [k for k in stats if match in k]
        if len(hits) == 1:
            avg = statistics.mean(stats[hits[0]])
            lines.append(f"achieved: {flops:.4e} FLOP / {avg / 1e6:.3f} ms = "
                         f"{flops / (avg * 1e-9) / 1e12:.1f} TFLOP/s ({hits[0][:40]}...)")
    return "\n".join(lines)


def main(argv=None):
    p = argparse.ArgumentParser(description="kernel duration stats of a rocprofv3 run")
    p.add_argument("folder")
    p.add_argument("--flops", type=float, default=None)
    p.add_argument("--match", default=None)
    p.add_argument("--skip", type=int, default=0,
                   help="drop the first N dispatches of every kernel (warmup steps)")
    args = p.parse_args(argv)
    print(render(skip_first(collect(args.folder), args.skip), args.flops, args.match))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
