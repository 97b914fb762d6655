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
summary for the same workload and tile, null when there is none), and
``cpu_baseline`` = the canonical FP32 formula timed on the host cores over a
bounded sample of the same workload (a few query rows of head 0 against all
keys; the oracle's CPU restatement, a reported baseline only).

``--causal top_left|bottom_right`` times the same workload under a causal
mask (not the headline metric): FLOPs then count only the (query, key)
pairs the mask leaves, 4*B*Hq*D*pairs.

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
                   help="approximate CPU time budget of the baseline sample")
    p.add_argument("--copy-mib", type=int, default=0,
                   help="after timing, run plain copies of this many MiB (counter calibration)")
    p.add_argument("--copy-reps", type=int, default=3)
    return p.parse_args(argv)


def traffic_from_profiles(workload_key):
    """HBM bytes per launch recorded in profiles/*_traffic.txt for this key, or None.

    The summaries hold a line ``key: <workload_key>`` and a line
    ``traffic_bytes_per_launch: <int>`` (FETCH_SIZE + WRITE_SIZE, each scaled
    by the copy-kernel calibration factor recorded beside it).
    """
    folder = os.path.join(REPO, "profiles")
    if not os.path.isdir(folder):
        return None
    for name in sorted(os.listdir(folder)):
        if not name.endswith("_traffic.txt"):
            continue
        fields = {}
        with open(os.path.join(folder, name), encoding="utf-8") as f:
            for line in f:
                key, sep, val = line.partition(":")
                if sep:
                    fields[key.strip()] = val.strip()
        if fields.get("key") == workload_key and "traffic_bytes_per_launch" in fields:
            return int(fields["traffic_bytes_per_launch"])
    return None


def cpu_baseline(case, cpu, budget_s):
    """Time the oracle's canonical FP32 formula on a sample of the workload.

    The sample is the first R query rows of (batch 0, head 0) against every
    key of that batch -- the same per-row work as the full problem, which is
    a sum of independent rows. R is sized from a probe run so that five or
    more timed runs fill about ``budget_s`` seconds of host time.
    """
    import torch

    from oracle.attention import attention_f32

    k, v = cpu["k"][:1, :1], cpu["v"][:1, :1]
    nk, d = k.shape[2], k.shape[3]
    cores = torch.get_num_threads()

    def run(rows):
        q = cpu["q"][:1, :1, :rows]
        t0 = time.perf_counter()
        attention_f32(q, k, v)
        return time.perf_counter() - t0

    probe_rows = 16
    run(probe_rows)                                # warmup
    per_row = run(probe_rows) / probe_rows
    rows = int(max(16, min(cpu["q"].shape[2], budget_s / 6 / per_row)) // 16 * 16)
    times = []
    start = time.perf_counter()
    while len(times) < 5 or (time.perf_counter() - start < budget_s and len(times) < 50):
        times.append(run(rows))
    med = statistics.median(times)
    flops = 4.0 * rows * nk * d
    return {
        "value": round(flops / med / 1e12, 5),
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "ms": round(med * 1e3, 2),
        "sample": f"{case.name}: {rows} query rows of batch 0 / head 0 against all {nk} keys "
                  f"(oracle.attention_f32, torch CPU FP32), median of {len(times)} runs "
                  f"after 1 warmup",
    }


def main(argv=None):
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(one GPU only; query tiles would shard across GPUs without communication)",
              file=sys.stderr)
        return 2

    import torch

    from fa_amd.core import registry
    from fa_amd.problem.canonical import build_canonical
    from fa_amd.problem.cases import CASES, visible_pairs

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    case = CASES[args.case]
    spec = registry.get(args.backend)
    bind = registry.prepare_call(spec, case)
    cpu = build_canonical(case, args.seed)
    canonical = {name: t.to("cuda") for name, t in cpu.items()}
    if args.no_cpu_baseline:
        cpu = None
    else:                                      # keep only what the CPU sample reads
        cpu = {"q": cpu["q"][:1, :1].clone(), "k": cpu["k"][:1, :1].clone(),
               "v": cpu["v"][:1, :1].clone()}
    call = bind(canonical)

    from fa_amd.backends import hip_common
    from fa_amd.binding import AttentionConfig, Operator

    acc = getattr(spec, "ACC", None)
    tile_name = None
    if acc is None and args.causal != "none":
        print(f"--causal needs a HIP backend, not {args.backend}", file=sys.stderr)
        return 2
    if acc is not None:
        op = Operator(hip_common.project(case, prebuilt=True).artifact_paths()[0],
                      AttentionConfig(acc=acc, kernel=args.kernel, causal=args.causal))
        tile_name = op.kernel_name(canonical["q"].shape, canonical["k"].shape)
        if args.kernel or args.causal != "none":
            # Explicit tile configuration (tuning runs) or a causal mask.
            call = lambda: op(canonical["q"], canonical["k"], canonical["v"])  # noqa: E731

    for _ in range(args.warmup):
        call()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(args.steps):
        call()
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
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

    workload_key = f"{args.backend} c{args.case} {case.name} tile={tile_name}"
    if args.causal != "none":
        workload_key += f" causal={args.causal}"
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
            "traffic": traffic_from_profiles(workload_key),
        },
        "cpu_baseline": None if cpu is None else cpu_baseline(case, cpu, args.cpu_seconds),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
