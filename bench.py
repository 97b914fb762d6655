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
``roofline`` against MI355X's dense FP16 MFMA peak, and ``cpu_baseline`` =
the canonical FP32 formula timed on the host cores at c0 (the oracle's CPU
restatement, a reported baseline only).

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
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="approximate CPU time budget of the baseline sample")
    return p.parse_args(argv)


def cpu_baseline(budget_s):
    """Time the oracle's canonical FP32 formula at c0 on the host cores."""
    import torch

    from fa_amd.problem.canonical import build_canonical
    from fa_amd.problem.cases import CASES, CPU_CASE
    from oracle.attention import attention_f32

    case = CASES[CPU_CASE]
    t = build_canonical(case, 0)
    cores = torch.get_num_threads()
    attention_f32(t["q"], t["k"], t["v"])          # warmup
    times = []
    start = time.perf_counter()
    while len(times) < 5 or (time.perf_counter() - start < budget_s and len(times) < 50):
        t0 = time.perf_counter()
        attention_f32(t["q"], t["k"], t["v"])
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {
        "value": round(case.flops / med / 1e12, 5),
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "ms": round(med * 1e3, 2),
        "sample": f"c0 {case.name}: full FP32 forward (oracle.attention_f32, torch CPU), "
                  f"median of {len(times)} runs after 1 warmup",
    }


def main(argv=None):
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the attention path shards without communication; see DESIGN.md)",
              file=sys.stderr)
        return 2

    import torch

    from fa_amd.core import registry
    from fa_amd.problem.canonical import build_canonical
    from fa_amd.problem.cases import CASES

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    case = CASES[args.case]
    spec = registry.get(args.backend)
    bind = registry.prepare_call(spec, case)
    canonical = build_canonical(case, args.seed, device="cuda")
    call = bind(canonical)
    if args.kernel:
        # Re-bind with an explicit tile configuration (tuning runs).
        from fa_amd.backends import hip_common
        from fa_amd.binding import AttentionConfig, Operator

        op = Operator(hip_common.project(case, prebuilt=True).artifact_paths()[0],
                      AttentionConfig(acc=spec.ACC, kernel=args.kernel))
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
    tflops = case.flops / (ms * 1e-3) / 1e12

    acc = getattr(spec, "ACC", "fp32")
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
            "workload": f"c{args.case} {case.name} non-causal GQA forward, {acc}-accumulate",
            "backend": args.backend,
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
            "traffic": None,
        },
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline(args.cpu_seconds),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
