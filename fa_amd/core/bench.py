"""Benchmark orchestrator across backends and cases (one GPU).

Phase A (CPU, parallel)   build every selected backend whose driver asks for
                          it, each in a runner subprocess that sees no GPU.
Phase B (GPU, in-process) per case: prepare every backend before any input
                          exists, draw the canonical inputs, warm each backend
                          up, time it (device time, ``profiler.profile_case_us``)
                          and check it against the reference backend.
Report                    long-format CSV + console table with average
                          microseconds, ratio to the reference, check verdict,
                          max |diff|, QK/PV TFLOP/s and % of the FP16 MFMA peak.

Mirrors the reference's ``core/bench.py:1-258``; the multi-card fan-out is
dropped (one GPU) and the timing uses HIP events rather than the NPU
profiler. Run as ``python -m fa_amd.core.bench``.
"""

import argparse
import csv
import os
import subprocess
import sys
from datetime import datetime

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))

import torch

from fa_amd.core import profiler, registry, schedule
from fa_amd.core.contract import KernelNameError
from fa_amd.problem.cases import CASES

REPO_ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
PEAK_FP16_TFLOPS = 2516.6


def _runner(*extra):
    return [sys.executable, "-m", "fa_amd.core.runner", *map(str, extra)]


# --------------------------------------------------------------------------- #
# Phase A: parallel compile
# --------------------------------------------------------------------------- #
def _compile_task(packed):
    """Run one backend build in a fresh CPU process (no GPU visible)."""
    backend, case_index = packed
    env = os.environ.copy()
    env["HIP_VISIBLE_DEVICES"] = ""
    env["CUDA_VISIBLE_DEVICES"] = ""
    cmd = _runner("--backend", backend, "--case-index", case_index, "--mode", "compile")
    r = subprocess.run(cmd, env=env, cwd=REPO_ROOT,
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    return backend, case_index, r.returncode, r.stdout


def compile_phase(backend_names, case_indices):
    tasks = []
    for name in backend_names:
        spec = registry.get(name)
        if not registry.needs_compile(spec):
            continue
        tasks.extend((name, i) for i in case_indices)
    if not tasks:
        return
    print(f">>> Phase A: compiling {len(tasks)} backend/case builds on CPU...")
    failed = []
    for backend, ci, rc, out in schedule.parallel_compile(tasks, _compile_task):
        tag = "ok" if rc == 0 else f"FAIL(rc={rc})"
        print(f"    {backend} {CASES[ci].name}: {tag}")
        if rc != 0:
            print(out)
            failed.append(f"{backend}/{CASES[ci].name}")
    if failed:
        raise RuntimeError(f"Compilation failed for {', '.join(failed)}")


# --------------------------------------------------------------------------- #
# Phase B: one case, in-process
# --------------------------------------------------------------------------- #
def process_case(case_index, *, backend_names, ref_name, iters, do_check, seed, atol, rtol):
    from fa_amd.problem.canonical import build_canonical

    case = CASES[case_index]
    prepared = {}
    skipped = set()
    for n in backend_names:
        try:
            prepared[n] = registry.prepare_call(registry.get(n), case)
        except KernelNameError:
            raise
        except Exception as e:  # a backend that cannot load is skipped, not fatal
            print(f"    [skip] {n}: {e}")
            skipped.add(n)
    canonical = build_canonical(case, seed, device="cuda")

    calls = {}
    for n in backend_names:
        if n in skipped:
            continue
        try:
            call = prepared[n](canonical)
            call()
            torch.cuda.synchronize()
            calls[n] = call
        except KernelNameError:
            raise
        except Exception as e:
            print(f"    [skip] {n}: {e}")
            skipped.add(n)

    times = profiler.profile_case_us(calls, backend_names, iters=iters)

    # Checks reuse the built callables; every operator must initialise its own
    # workspace, the harness never zeroes device memory for it.
    checks = {}
    if do_check:
        ref_out = None
        ordered = sorted(backend_names, key=lambda n: not registry.get(n).META.is_reference)
        for n in ordered:
            if n in skipped:
                checks[n] = ("ref", 0.0) if registry.get(n).META.is_reference else ("ERR", None)
                continue
            out = calls[n]().float()
            torch.cuda.synchronize()
            if registry.get(n).META.is_reference:
                ref_out = out.clone()
                checks[n] = ("ref", 0.0)
            elif ref_out is not None:
                max_diff = (out - ref_out).abs().max().item()
                try:
                    torch.testing.assert_close(out, ref_out, atol=atol, rtol=rtol)
                    checks[n] = ("PASS", max_diff)
                except AssertionError:
                    checks[n] = ("FAIL", max_diff)
            else:
                checks[n] = ("ERR", None)

    ref_us = times.get(ref_name)
    rows = []
    for n in backend_names:
        meta = registry.get(n).META
        us = times.get(n)
        ratio = f"{(us / ref_us) * 100:.1f}%" if (us and ref_us) else "N/A"
        tflops = case.flops / (us * 1e-6) / 1e12 if us else None
        status, diff = checks.get(n, ("skip", None))
        rows.append([case.name, n, "ref" if meta.is_reference else "",
                     f"{us:.2f}" if us else "N/A", ratio, status,
                     f"{diff:.5f}" if diff is not None else "N/A",
                     f"{tflops:.1f}" if tflops else "N/A",
                     f"{100 * tflops / PEAK_FP16_TFLOPS:.1f}%" if tflops else "N/A"])
    print(f"[done] {case.name:<24} " +
          " ".join(f"{n}={times[n]:.1f}us" if times.get(n) else f"{n}=N/A" for n in backend_names))
    return rows


# --------------------------------------------------------------------------- #
def _parse_cases(spec):
    spec = spec.strip()
    if spec == "all":
        return list(range(len(CASES)))
    out = []
    for tok in spec.split(","):
        tok = tok.strip()
        if not tok:
            continue
        try:
            i = int(tok)
        except ValueError:
            raise SystemExit(f"--cases: '{tok}' is not an integer index or 'all'")
        if not (0 <= i < len(CASES)):
            raise SystemExit(f"--cases: index {i} out of range 0..{len(CASES) - 1}")
        if i not in out:
            out.append(i)
    if not out:
        raise SystemExit("--cases: no valid case indices given")
    return out


HEADERS = ["Case", "Backend", "Ref", "Avg_us", "vs_ref", "Check", "MaxDiff", "TFLOPS", "PctPeak"]


def main(argv=None):
    p = argparse.ArgumentParser(description="benchmark orchestrator")
    p.add_argument("--backends", type=str, default=None,
                   help="comma-separated backend names (default: all registered)")
    p.add_argument("--cases", type=str, default="0",
                   help="'all' or comma-separated case indices (see --list-cases)")
    p.add_argument("--list-cases", action="store_true")
    p.add_argument("--iters", type=int, default=20)
    p.add_argument("--logdir", type=str, default=os.path.join(REPO_ROOT, "results"))
    p.add_argument("--no-check", action="store_true")
    p.add_argument("--no-compile", action="store_true")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--atol", type=float, default=1e-2)
    p.add_argument("--rtol", type=float, default=1e-2)
    args = p.parse_args(argv)

    if args.list_cases:
        for i, c in enumerate(CASES):
            print(f"{i:2d}  {c.name}")
        return 0

    backend_names = args.backends.split(",") if args.backends else registry.all_names()
    for name in backend_names:
        registry.require_attention(registry.get(name))
    ref_name, _ = registry.get_reference()
    if ref_name not in backend_names:
        backend_names = [ref_name] + backend_names

    case_indices = _parse_cases(args.cases)
    stamp = datetime.now().strftime("%Y%m%d_%H%M%S")
    label = "all" if args.cases.strip() == "all" else "sel" + "_".join(map(str, case_indices))
    session_dir = os.path.join(args.logdir, f"bench_{label}_{stamp}")
    os.makedirs(session_dir, exist_ok=True)
    print(f">>> backends={backend_names} ref={ref_name}")
    print(f">>> cases: {case_indices}; session: {session_dir}")

    if not args.no_compile:
        compile_phase(backend_names, case_indices)

    rows = []
    for ci in case_indices:
        rows.extend(process_case(ci, backend_names=backend_names, ref_name=ref_name,
                                 iters=args.iters, do_check=not args.no_check,
                                 seed=args.seed, atol=args.atol, rtol=args.rtol))

    csv_path = os.path.join(session_dir, "report.csv")
    with open(csv_path, "w", newline="", encoding="utf-8") as f:
        w = csv.writer(f)
        w.writerow(HEADERS)
        w.writerows(rows)
    print("\n" + "  ".join(HEADERS))
    for r in rows:
        print("  ".join(str(x) for x in r))
    print(f"\n[done] report -> {csv_path}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
