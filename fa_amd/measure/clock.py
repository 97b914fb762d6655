"""Running shader clock of a kernel, from its trace records.

The attention kernel's trace mode (``fa_fwd_trace``) writes one record of 8
uint64 words per 256-row query tile, the MFMA ceiling kernel one per
workgroup: words 1/2 are ``s_memrealtime`` (a constant 100 MHz reference
clock) at the start and after the main loop, words 3/4 ``s_memtime``
(shader-clock cycles) at the same points. ``summarize`` turns the records
into the clock each tile or workgroup ran at,
``(w4 - w3) / (w2 - w1) * 100 MHz``, and its spread over the launch and over
the 8 accelerator dies (XCC_ID, word 0 bits 32-35, attention kernel only).

``python -m fa_amd.measure.clock`` runs the attention forward of one
configuration on the GPU: warmup forwards (so the board reaches its
steady-state clock), timed production forwards, then one trace-mode forward,
and prints the clock summary together with the MFMA roof at that clock:
256 CUs x 4096 FLOP/clk x f, against which the achieved rate is compared.
"""

from __future__ import annotations

import argparse
import os
import sys

import numpy as np

REF_CLOCK_MHZ = 100.0
PEAK_TFLOPS = 2516.6
PEAK_CLOCK_MHZ = 2400.0


def clocks_mhz(records) -> np.ndarray:
    """Shader clock (MHz) of each record with a nonzero time span."""
    r = np.asarray(records, dtype=np.int64).reshape(-1, 8)
    real = (r[:, 2] - r[:, 1]).astype(np.float64)
    cyc = (r[:, 4] - r[:, 3]).astype(np.float64)
    ok = real > 0
    return cyc[ok] / real[ok] * REF_CLOCK_MHZ


def summarize(records) -> dict:
    r = np.asarray(records, dtype=np.int64).reshape(-1, 8)
    mhz = clocks_mhz(r)
    if mhz.size == 0:
        raise ValueError("no trace record spans a nonzero time")
    xcc = (r[:, 0] >> 32) & 15
    real = r[:, 2] - r[:, 1]
    per_xcc = {int(x): float(np.median(clocks_mhz(r[xcc == x]))) for x in sorted(set(xcc.tolist()))
               if np.any((xcc == x) & (real > 0))}
    weights = real[real > 0].astype(np.float64)
    return {
        "records": int(r.shape[0]),
        "median_mhz": float(np.median(mhz)),
        "mean_mhz_time_weighted": float(np.sum(mhz * weights) / np.sum(weights)),
        "p10_mhz": float(np.percentile(mhz, 10)),
        "p90_mhz": float(np.percentile(mhz, 90)),
        "min_mhz": float(mhz.min()),
        "max_mhz": float(mhz.max()),
        "per_xcc_median_mhz": per_xcc,
        "span_ms": float((r[:, 2].max() - r[:, 1].min()) / (REF_CLOCK_MHZ * 1e3)),
        "record_ms_median": float(np.median(real) / (REF_CLOCK_MHZ * 1e3)),
    }


def roof_at(mhz: float) -> float:
    """Dense FP16 MFMA rate (TFLOP/s) of the whole chip at shader clock ``mhz``."""
    return PEAK_TFLOPS * mhz / PEAK_CLOCK_MHZ


def render(title, s, achieved_tflops=None) -> list:
    lines = [title,
             f"records: {s['records']}",
             f"clock_mhz: median {s['median_mhz']:.0f}, time-weighted mean "
             f"{s['mean_mhz_time_weighted']:.0f}, p10 {s['p10_mhz']:.0f}, p90 {s['p90_mhz']:.0f}, "
             f"min {s['min_mhz']:.0f}, max {s['max_mhz']:.0f}",
             f"span_ms: {s['span_ms']:.3f} (first entry to last loop end), "
             f"per-record median {s['record_ms_median']:.3f}"]
    if s["per_xcc_median_mhz"]:
        lines.append("per_xcc_median_mhz: " + ", ".join(
            f"{x}: {v:.0f}" for x, v in s["per_xcc_median_mhz"].items()))
    roof = roof_at(s["mean_mhz_time_weighted"])
    lines.append(f"mfma_roof_at_clock_tflops: {roof:.1f} (2516.6 x f / 2400 MHz)")
    if achieved_tflops:
        lines.append(f"achieved_tflops: {achieved_tflops:.1f} -> {achieved_tflops / roof:.3f} of the "
                     f"roof at the running clock, {achieved_tflops / PEAK_TFLOPS:.3f} of the "
                     f"nominal peak")
    return lines


def run_attention(case_index, acc, warmup, steps, seed=0):
    """(achieved TFLOP/s of the production forward, trace records, trace-mode TFLOP/s)."""
    import torch

    from fa_amd.backends import hip_common
    from fa_amd.harness import timing
    from fa_amd.problem.canonical import build_canonical
    from fa_amd.problem.cases import CASES

    case = CASES[case_index]
    x = build_canonical(case, seed, device="cuda")
    run = hip_common.operator(acc, case)
    traced = hip_common.operator(acc, case, trace=True)
    args = (x["q"], x["k"], x["v"])
    us = timing.device_us(lambda: run(*args), iters=steps, warmup=warmup)
    us_trace = timing.device_us(lambda: traced(*args), iters=1, warmup=0)
    records = traced.last["trace"].cpu().numpy()
    return case.flops / us / 1e6, records, case.flops / us_trace / 1e6


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--case", type=int, default=3)
    ap.add_argument("--acc", default="fp32", choices=("fp32", "fp16"))
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--out", help="also write the summary to this file")
    ap.add_argument("--command", default="", help="command line recorded in the summary")
    ap.add_argument("--records", help="also save the raw trace records (.npy)")
    args = ap.parse_args(argv)
    repo = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    if repo not in sys.path:
        sys.path.insert(0, repo)
    from fa_amd.problem.cases import CASES

    tflops, records, tflops_trace = run_attention(args.case, args.acc, args.warmup, args.steps)
    if args.records:
        np.save(args.records, records)
    s = summarize(records)
    lines = render(f"# running shader clock of hip_fa_{args.acc}acc at c{args.case} "
                   f"{CASES[args.case].name} (trace-mode records)", s, tflops)
    lines.insert(1, f"command: {args.command or 'python -m fa_amd.measure.clock ' + ' '.join(argv or sys.argv[1:])}")
    lines.append(f"trace_mode_forward_tflops: {tflops_trace:.1f} (one forward, the stamped kernel)")
    print("\n".join(lines), flush=True)
    if args.out:
        with open(args.out, "w", encoding="utf-8") as f:
            f.write("\n".join(lines) + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
