"""HBM traffic per kernel launch from two rocprofv3 counter runs.

``FETCH_SIZE`` and ``WRITE_SIZE`` (KiB per dispatch, summed over the L2
channels) are collected in separate ``rocprofv3 --pmc`` passes of the same
bench command, which also runs a calibration kernel of known size
(``bench.py --copy-mib M``: ``bitwise_not`` over M MiB, reading M MiB and
writing M MiB). Each counter of the attention kernel is scaled by
known bytes / counter bytes of the calibration kernel, and the two scaled
figures are added: ``traffic_bytes_per_launch``. The summary file this writes
under ``profiles/`` is what ``bench.py`` reports as ``roofline.traffic``.

The algorithmic bytes of a launch, against which the traffic is compared,
come from the configuration (``--case i``): Q and O (B*Hq*Nq*128 FP16 each)
plus K and V (B*Hkv*Nk*128 FP16 each), every tensor read or written once.

Usage (on the CPU, after the GPU runs):
  python -m fa_amd.measure.traffic --fetch DIR --write DIR --copy-mib M \\
      --case 3 --key "<backend> c<i> <case> tile=<tile>" --command-fetch "..." \\
      --command-write "..." --out profiles/<name>_traffic.txt
"""

import argparse
import collections
import csv
import glob
import os
import statistics


def per_dispatch(folder, counter):
    """{kernel name: [value per dispatch]} for one counter of a rocprofv3 CSV run."""
    paths = glob.glob(os.path.join(folder, "**", "*counter_collection.csv"), recursive=True)
    if not paths:
        raise FileNotFoundError(f"no counter_collection.csv under {folder}")
    sums = collections.defaultdict(float)
    names = {}
    for path in paths:
        with open(path, newline="", encoding="utf-8") as f:
            for row in csv.DictReader(f):
                if row["Counter_Name"] != counter:
                    continue
                key = (path, row["Dispatch_Id"])
                sums[key] += float(row["Counter_Value"])
                names[key] = row["Kernel_Name"]
    out = collections.defaultdict(list)
    for key, val in sums.items():
        out[names[key]].append(val)
    return dict(out)


def pick(kernels, needle):
    hits = [k for k in kernels if needle in k]
    if len(hits) != 1:
        raise ValueError(f"expected one kernel containing {needle!r}, found {hits}")
    return hits[0]


def summarize(fetch_dir, write_dir, copy_mib, attn_needle="hip_fa_", copy_needle="bitwise_not"):
    fetch = per_dispatch(fetch_dir, "FETCH_SIZE")
    write = per_dispatch(write_dir, "WRITE_SIZE")
    attn_f, copy_f = pick(fetch, attn_needle), pick(fetch, copy_needle)
    attn_w, copy_w = pick(write, attn_needle), pick(write, copy_needle)
    known = copy_mib * (1 << 20)
    fetch_kib = statistics.median(fetch[attn_f])
    write_kib = statistics.median(write[attn_w])
    copy_fetch_kib = statistics.median(fetch[copy_f])
    copy_write_kib = statistics.median(write[copy_w])
    f_factor = known / (copy_fetch_kib * 1024)
    w_factor = known / (copy_write_kib * 1024)
    return {
        "attention_kernel": attn_f,
        "fetch_kib": fetch_kib,
        "write_kib": write_kib,
        "fetch_dispatches": len(fetch[attn_f]),
        "write_dispatches": len(write[attn_w]),
        "copy_kernel": copy_f,
        "copy_bytes": known,
        "copy_fetch_kib": copy_fetch_kib,
        "copy_write_kib": copy_write_kib,
        "fetch_factor": f_factor,
        "write_factor": w_factor,
        "fetch_bytes": fetch_kib * 1024 * f_factor,
        "write_bytes": write_kib * 1024 * w_factor,
    }


def algorithmic_bytes(case):
    """Bytes a launch must move at least: Q, K, V read and O written once (FP16)."""
    q_o = case.batch * case.heads_q * case.seq_len * case.dim * 2
    k_v = case.batch * case.heads_kv * case.seq_len * case.dim * 2
    return 2 * q_o + 2 * k_v


def main(argv=None):
    p = argparse.ArgumentParser(description="HBM bytes per launch from FETCH_SIZE/WRITE_SIZE runs")
    p.add_argument("--fetch", required=True)
    p.add_argument("--write", required=True)
    p.add_argument("--copy-mib", type=int, required=True)
    p.add_argument("--key", required=True)
    p.add_argument("--case", type=int, required=True,
                   help="configuration index c0..c4 (its Q+K+V+O bytes are the algorithmic bytes)")
    p.add_argument("--command-fetch", default="")
    p.add_argument("--command-write", default="")
    p.add_argument("--session", default="",
                   help="which profiling run the passes come from (bench.py names it beside the value)")
    p.add_argument("--out", required=True)
    args = p.parse_args(argv)
    s = summarize(args.fetch, args.write, args.copy_mib)
    total = int(round(s["fetch_bytes"] + s["write_bytes"]))
    from fa_amd.problem.cases import CASES

    algo = algorithmic_bytes(CASES[args.case])
    lines = [
        "# HBM traffic per launch (rocprofv3 FETCH_SIZE and WRITE_SIZE, separate passes)",
        f"key: {args.key}",
    ]
    if args.session:
        lines.append(f"session: {args.session}")
    lines += [
        f"command_fetch: {args.command_fetch}",
        f"command_write: {args.command_write}",
        f"attention_kernel: {s['attention_kernel']}",
        f"attention_FETCH_SIZE_KiB_per_dispatch: {s['fetch_kib']:.0f} (median of {s['fetch_dispatches']})",
        f"attention_WRITE_SIZE_KiB_per_dispatch: {s['write_kib']:.0f} (median of {s['write_dispatches']})",
        f"calibration_kernel: {s['copy_kernel']}",
        f"calibration_bytes_read_and_written: {s['copy_bytes']}",
        f"calibration_FETCH_SIZE_KiB: {s['copy_fetch_kib']:.0f} -> factor {s['fetch_factor']:.4f}",
        f"calibration_WRITE_SIZE_KiB: {s['copy_write_kib']:.0f} -> factor {s['write_factor']:.4f}",
        f"fetch_bytes_per_launch: {s['fetch_bytes']:.0f}",
        f"write_bytes_per_launch: {s['write_bytes']:.0f}",
        f"traffic_bytes_per_launch: {total}",
    ]
    lines.append(f"algorithmic_bytes_per_launch: {algo} (Q + K + V + O of c{args.case}; "
                 f"traffic / algorithmic = {total / algo:.3f})")
    os.makedirs(os.path.dirname(os.path.abspath(args.out)), exist_ok=True)
    with open(args.out, "w", encoding="utf-8") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
