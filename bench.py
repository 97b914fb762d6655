"""Benchmark of the MI355X flash-attention forward (one JSON line on stdout).

A step is one forward of the selected backend over one batch of the workload:
by default the headline configuration c3 (B=2, Nq=Nk=131072, Hq=12, Hkv=1,
D=128, FP16 in/out, FP32-accumulated O), inputs resident in HBM before the
timed region. W warmup steps run untimed, then exactly K steps are timed with
HIP events on the stream the kernels are launched on (torch's current
stream), bracketed by ``torch.cuda.synchronize()``.

Reported, mirroring the reference's metric (``README.md:86-88``: QK/PV FLOPs
= 4*B*Hq*Nq*Nk*D over the forward time, as a fraction of the FP16 matrix
peak): ``value`` = QK/PV TFLOP/s, ``ms_per_step`` = forward milliseconds,
``roofline`` against MI355X's dense FP16 MFMA peak (``traffic`` = HBM bytes
per attention launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
summary for the same workload and tile, null when there is none; it is not
measured in this run, and ``traffic_source`` names the summary file and the
session it records), and
``cpu_baseline`` = the canonical FP32 formula (the oracle's CPU
restatement) timed on every host core over the full c0 forward, the
CPU-runnable plumbing configuration (a reported baseline only).

``--causal top_left|bottom_right`` times the same workload under a causal
mask (not the headline metric): FLOPs then count only the (query, key)
pairs the mask leaves, 4*B*Hq*D*pairs.

``clock`` (HIP backends) is the shader clock the attention kernel ran at,
from one trace-mode forward after the timed region, with the MFMA roof at
that clock; ``sustained`` is the board's sustained dense FP16 matrix rate
measured in the same process (torch FP16 GEMMs, an MFMA-only loop, the
same loop with LDS operands and the softmax's VALU mix, and the attention
kernel's ping-pong skeleton with its softmax step but no data to stage,
``fa_amd.measure.ceiling``), with ``value`` as a fraction of each.

``configs`` (HIP backends, full attention) times the configurations
``--configs`` (default all of c0..c4; ``--configs ""`` for none) with both
accumulation variants after the headline, in the same process: canonical
inputs, ``--config-warmup`` untimed and ``--config-steps`` timed forwards
each, HIP events around the timed ones (the headline's own entry is the
headline measurement).

``--copy-mib M`` additionally runs ``--copy-reps`` plain device-to-device
copies of M MiB after the timed region, untimed: the calibration kernel the
traffic summary scales the FETCH_SIZE and WRITE_SIZE counters by.

One GPU only: ``--gpus`` above 1 exits with a message.
"""

import argparse
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

# 256 CUs x 2.4 GHz x 4096 FP16 FLOP/clk/CU (dense MFMA).
PEAK_FP16_TFLOPS = 2516.6


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--case", type=int, default=3, help="configuration index c0..c4")
    p.add_argument("--backend", default="hip_fa_fp32acc")
    p.add_argument("--kernel", type=int, default=0, help="tile configuration (0 = automatic)")
    p.add_argument("--causal", default="none", choices=("none", "top_left", "bottom_right"),
                   help="attention mask (the headline workload is full attention)")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="host time budget of the CPU baseline's timed runs")
    p.add_argument("--copy-mib", type=int, default=0,
                   help="after timing, run plain copies of this many MiB (counter calibration)")
    p.add_argument("--copy-reps", type=int, default=3)
    p.add_argument("--no-ceiling", action="store_true",
                   help="skip the sustained-rate (GEMM and MFMA loop) and clock measurements")
    p.add_argument("--configs", default="0,1,2,3,4",
                   help="configurations to time with both accumulation variants ('' = none)")
    p.add_argument("--config-steps", type=int, default=5)
    p.add_argument("--config-warmup", type=int, default=2)
    return p.parse_args(argv)


def time_forward(call, steps, warmup):
    """Milliseconds per call: ``warmup`` untimed calls, then ``steps`` calls
    between HIP events on torch's current stream (where the kernels run)."""
    import torch

    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        call()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def config_table(indices, steps, warmup, headline=None, inputs=None):
    """{"c<i>": {"fp32": {...}, "fp16": {...}}} over configurations ``indices``:
    ms per forward, QK/PV TFLOP/s and percent of the FP16 peak, full
    attention. ``headline`` = (case index, acc, ms) is entered as measured;
    ``inputs`` = (case index, canonical tensors on the GPU) are reused."""
    import torch

    from fa_amd.backends import hip_common
    from fa_amd.problem.canonical import build_canonical
    from fa_amd.problem.cases import CASES

    table = {}
    for i in indices:
        case = CASES[i]
        x = inputs[1] if inputs is not None and inputs[0] == i else None
        row = {}
        for acc in ("fp32", "fp16"):
            if headline is not None and headline[:2] == (i, acc):
                ms = headline[2]
            else:
                if x is None:
                    x = build_canonical(case, 0, device="cuda")
                op = hip_common.operator(acc, case)
                ms = time_forward(lambda: op(x["q"], x["k"], x["v"]), steps, warmup)
                del op
            tflops = case.flops / (ms * 1e-3) / 1e12
            row[acc] = {"ms": round(ms, 4), "tflops": round(tflops, 1),
                        "pct_peak": round(100 * tflops / PEAK_FP16_TFLOPS, 2)}
        row["workload"] = case.name
        table[f"c{i}"] = row
        del x
        torch.cuda.empty_cache()
    return table


def traffic_record(workload_key):
    """(bytes, source) of the HBM traffic per launch committed for this key, or (None, None).

    The summaries ``profiles/*_traffic.txt`` hold a line ``key:
    <workload_key>``, a line ``traffic_bytes_per_launch: <int>`` (FETCH_SIZE +
    WRITE_SIZE, each scaled by the copy-kernel calibration factor recorded
    beside it) and optionally ``session: <text>`` naming the profiling run;
    ``source`` names the file and that session, since the value comes from a
    separate counter run and not from the timed region.
    """
    folder = os.path.join(REPO, "profiles")
    if not os.path.isdir(folder):
        return None, None
    for name in sorted(os.listdir(folder)):
        if not name.endswith("_traffic.txt"):
            continue
        fields = {}
        with open(os.path.join(folder, name), encoding="utf-8") as f:
            for line in f:
                key, sep, val = line.partition(":")
                if sep:
                    fields.setdefault(key.strip(), val.strip())
        if fields.get("key") == workload_key and "traffic_bytes_per_launch" in fields:
            source = (f"profiles/{name}: rocprofv3 FETCH_SIZE and WRITE_SIZE passes of a "
                      f"separate profiling run, not measured in this run")
            if fields.get("session"):
                source += f" ({fields['session']})"
            return int(fields["traffic_bytes_per_launch"]), source
    return None, None


def traffic_from_profiles(workload_key):
    """HBM bytes per launch recorded in profiles/*_traffic.txt for this key, or None."""
    return traffic_record(workload_key)[0]


def cpu_baseline(min_runs=5, budget_s=12.0):
    """Time the canonical FP32 formula on the host for the full c0 forward.

    The CPU-runnable plumbing configuration c0 (B=1, Hq=12, Hkv=1, N=4096,
    D=128, 1.03e11 FLOP) run whole through ``oracle.attention_f32`` (the
    canonical ``softmax(q k^T * scale) v`` in FP32 torch on the CPU) with
    ``torch.set_num_threads(os.cpu_count())``: one warmup run, then the
    median of at least ``min_runs`` runs (more while they fit in
    ``budget_s`` seconds, at most 25). A reported baseline, not a target.
    """
    import torch

    from fa_amd.problem.canonical import build_canonical
    from fa_amd.problem.cases import CASES, CPU_CASE
    from oracle.attention import attention_f32

    case = CASES[CPU_CASE]
    cores = os.cpu_count() or 1
    threads_before = torch.get_num_threads()
    torch.set_num_threads(cores)
    try:
        x = build_canonical(case, seed=0)
        attention_f32(x["q"], x["k"], x["v"])               # warmup
        times = []
        start = time.perf_counter()
        while len(times) < min_runs or (time.perf_counter() - start < budget_s and len(times) < 25):
            t0 = time.perf_counter()
            attention_f32(x["q"], x["k"], x["v"])
            times.append(time.perf_counter() - t0)
    finally:
        torch.set_num_threads(threads_before)
    med = statistics.median(times)
    return {
        "value": round(case.flops / med / 1e12, 5),
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "ms": round(med * 1e3, 2),
        "gflops": round(case.flops / med / 1e9, 1),
        "sample": f"c0 {case.name}: the full forward ({case.flops:.3e} FLOP) through "
                  f"oracle.attention_f32 (torch CPU FP32, {cores} threads), median of "
                  f"{len(times)} runs after 1 warmup",
    }


def main(argv=None):
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(one GPU only; query tiles would shard across GPUs without communication)",
              file=sys.stderr)
        return 2

    import torch

    from fa_amd.harness.catalog import Catalog
    from fa_amd.problem.canonical import build_canonical
    from fa_amd.problem.cases import CASES, visible_pairs

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    case = CASES[args.case]
    catalog = Catalog.default()
    entry = catalog.attention(args.backend)
    bind = catalog.prepare(args.backend, case)
    canonical = build_canonical(case, args.seed, device="cuda")
    call = bind(canonical)

    from fa_amd.backends import hip_common

    acc = getattr(entry.module, "ACC", None)
    tile_name = None
    if acc is None and args.causal != "none":
        print(f"--causal needs a HIP backend, not {args.backend}", file=sys.stderr)
        return 2
    if acc is not None:
        op = hip_common.operator(acc, case, kernel=args.kernel, causal=args.causal)
        tile_name = op.kernel_name(canonical["q"].shape, canonical["k"].shape)
        if args.kernel or args.causal != "none":
            # Explicit tile configuration (tuning runs) or a causal mask.
            call = lambda: op(canonical["q"], canonical["k"], canonical["v"])  # noqa: E731

    ms = time_forward(call, args.steps, args.warmup)
    flops = (4 * case.batch * case.heads_q * case.dim
             * visible_pairs(case.seq_len, case.seq_len, args.causal))
    tflops = flops / (ms * 1e-3) / 1e12

    if args.copy_mib:
        n = args.copy_mib << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda").random_(0, 255)
        dst = torch.empty_like(src)
        for _ in range(args.copy_reps):
            # An elementwise kernel that reads n bytes and writes n bytes
            # (a plain copy_ may go to a DMA engine the counters do not see).
            torch.bitwise_not(src, out=dst)
        torch.cuda.synchronize()
        del src, dst

    # After the timed region (untimed): the running clock from one trace-mode
    # forward of the same tile, and the board's sustained matrix rate.
    clock_line, sustained = None, None
    if not args.no_ceiling:
        from fa_amd.measure import ceiling, clock

        if acc is not None:
            traced = hip_common.operator(acc, case, kernel=args.kernel, causal=args.causal,
                                         trace=True)
            traced(canonical["q"], canonical["k"], canonical["v"])
            torch.cuda.synchronize()
            s = clock.summarize(traced.last["trace"].cpu().numpy())
            f = s["mean_mhz_time_weighted"]
            clock_line = {"median_mhz": round(s["median_mhz"], 1), "mean_mhz": round(f, 1),
                          "p10_mhz": round(s["p10_mhz"], 1), "p90_mhz": round(s["p90_mhz"], 1),
                          "mfma_roof_at_clock": round(clock.roof_at(f), 1),
                          "frac_at_clock": round(tflops / clock.roof_at(f), 4),
                          "source": "fa_fwd_trace records (s_memtime / s_memrealtime per query tile)"}
            del traced
        sustained = ceiling.measure(gemm_reps=10)
        sustained["frac_of_gemm"] = round(tflops / sustained["gemm_best_tflops"], 4)
        sustained["frac_of_mfma_loop"] = round(tflops / sustained["mfma_loop_best_tflops"], 4)
        sustained["frac_of_softmax_mix_loop"] = round(
            tflops / sustained["softmax_mix_loop_tflops"], 4)
        if "skeleton_tflops" in sustained:
            sustained["frac_of_skeleton"] = round(tflops / sustained["skeleton_tflops"], 4)

    configs = None
    indices = [int(c) for c in args.configs.split(",") if c.strip()]
    if acc is not None and indices:
        same = args.causal == "none" and not args.kernel and args.seed == 0
        headline = (args.case, acc, ms) if same else None
        inputs = (args.case, canonical) if args.seed == 0 else None
        del call, bind
        configs = config_table(indices, args.config_steps, args.config_warmup, headline, inputs)

    workload_key = f"{args.backend} c{args.case} {case.name} tile={tile_name}"
    if args.causal != "none":
        workload_key += f" causal={args.causal}"
    traffic, traffic_source = traffic_record(workload_key)
    mask = "non-causal" if args.causal == "none" else f"causal ({args.causal})"
    line = {
        "metric": "fwd ms & QK/PV TFLOPS (% FP16 MFMA peak), B=2 N=131072 Hq=12 D=128",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {
            "workload": f"c{args.case} {case.name} {mask} GQA forward, "
                        f"{acc or 'fp32'}-accumulate",
            "causal": args.causal,
            "backend": args.backend,
            "tile": tile_name,
            "batch": case.batch, "seq_len": case.seq_len, "heads_q": case.heads_q,
            "heads_kv": case.heads_kv, "dim": case.dim, "dist": case.dist,
            "kernel": args.kernel, "parallelism": "none",
        },
        "pct_peak": round(100 * tflops / PEAK_FP16_TFLOPS, 2),
        "roofline": {
            "bound": "mfma",
            "achieved": round(tflops, 2),
            "peak": PEAK_FP16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(tflops / PEAK_FP16_TFLOPS, 4),
            "traffic": traffic,
            "traffic_source": traffic_source,
        },
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline(budget_s=args.cpu_seconds),
        "clock": clock_line,
        "sustained": sustained,
        "configs": configs,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
