"""Command line of the harness: ``python -m fa_amd.harness <command>``.

  list                         the configurations (c0..c4) and the backends
  check --backend B --case C   one backend against the reference; prints
                               ``CHECK <case> backend=<B> PASS|FAIL max_abs_diff=...``,
                               exit status 0 on PASS, 1 on FAIL
  build [--backend B]          run the build step of every (or one) backend
                               that has one, on the CPU
  report --cases C,... [--backends B,...] [--iters N] [--out report.csv]
                               timing + check table per configuration
  kernels <rocprofv3 dir> [--backends B,...] [--skip N] [--unowned N]
                               each backend's mean device-kernel duration in a
                               ``rocprofv3 --kernel-trace`` run (for example of
                               ``report``), attributed by the reference
                               profiler's kernel-name rule; kernels no backend
                               owns (the HIP prep kernel) are listed apart

Configurations are named ``c0``..``c4`` (this repository's table, which
begins with the CPU-sized c0) or by their full case name
(``B2_S131072_Q12_KV1_D128``); note that the reference's ``--case-index``
counts from its own first case, B2 N131072, which is c3 here.
"""

from __future__ import annotations

import argparse
import os
import sys

REPO = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def resolve_cases(spec: str):
    from fa_amd.problem.cases import CASES

    if spec.strip() == "all":
        return list(CASES)
    by_name = {c.name: c for c in CASES}
    chosen = []
    for token in filter(None, (t.strip() for t in spec.split(","))):
        if token[:1] == "c" and token[1:].isdigit() and int(token[1:]) < len(CASES):
            case = CASES[int(token[1:])]
        elif token in by_name:
            case = by_name[token]
        else:
            raise SystemExit(f"unknown configuration {token!r}: use c0..c{len(CASES) - 1}, "
                             "a case name, or 'all'")
        if case not in chosen:
            chosen.append(case)
    if not chosen:
        raise SystemExit("no configuration selected")
    return chosen


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m fa_amd.harness", description=__doc__.splitlines()[0])
    sub = ap.add_subparsers(dest="command", required=True)
    sub.add_parser("list")
    p_check = sub.add_parser("check")
    p_check.add_argument("--backend", required=True)
    p_check.add_argument("--case", required=True)
    p_build = sub.add_parser("build")
    p_build.add_argument("--backend")
    p_rep = sub.add_parser("report")
    p_rep.add_argument("--cases", default="c0")
    p_rep.add_argument("--backends")
    p_rep.add_argument("--iters", type=int, default=20)
    p_rep.add_argument("--no-check", action="store_true")
    p_rep.add_argument("--out")
    p_ker = sub.add_parser("kernels")
    p_ker.add_argument("trace_dir")
    p_ker.add_argument("--backends")
    p_ker.add_argument("--skip", type=int, default=0,
                       help="drop the first N dispatches of every kernel (warmup calls)")
    p_ker.add_argument("--unowned", type=int, default=5,
                       help="list this many unowned kernels (by device time), then their total")
    for p in (p_check, p_rep):
        p.add_argument("--seed", type=int, default=0)
        p.add_argument("--atol", type=float, default=1e-2)
        p.add_argument("--rtol", type=float, default=1e-2)
    args = ap.parse_args(argv)

    from fa_amd.harness import report
    from fa_amd.harness.catalog import Catalog

    catalog = Catalog.default()
    if args.command == "list":
        from fa_amd.problem.cases import CASES

        for i, c in enumerate(CASES):
            print(f"c{i}  {c.name}")
        for n in catalog.names(include_diagnostic=True):
            meta = catalog[n].meta
            tag = " (reference)" if meta.is_reference else ""
            print(f"backend {n}: type={meta.type}{tag}")
        return 0
    if args.command == "build":
        names = [args.backend] if args.backend else catalog.names()
        from fa_amd.problem.cases import CASES

        for n in names:
            built = catalog.build(n, CASES[0])
            print(f"BUILD {n} {'done' if built else 'nothing to build'}")
        return 0

    if args.command == "kernels":
        from fa_amd.harness.timing import KernelOwners, kernel_table, render_kernel_table

        names = args.backends.split(",") if args.backends else catalog.names()
        owners = KernelOwners(names, op_types={n: catalog[n].meta.op_type for n in names})
        table, unowned = kernel_table(args.trace_dir, owners, skip=args.skip)
        print(render_kernel_table(table, unowned, args.unowned))
        return 0

    tol = report.Tolerance(args.atol, args.rtol)
    if args.command == "check":
        (case,) = resolve_cases(args.case)
        passed, diff = report.check_backend(catalog, args.backend, case, seed=args.seed, tol=tol)
        print(report.check_line(case, args.backend, passed, diff, tol), flush=True)
        return 0 if passed else 1

    names = args.backends.split(",") if args.backends else catalog.names()
    for n in names:
        catalog.attention(n)
    rows = []
    for case in resolve_cases(args.cases):
        rows.extend(report.run_case(catalog, case, names, iters=args.iters, seed=args.seed,
                                    tol=tol, do_check=not args.no_check))
        print(f"[case] {case.name} done", flush=True)
    widths = [max(len(h), *(len(r.cells()[i]) for r in rows)) for i, h in enumerate(report.HEADERS)]
    print("  ".join(h.ljust(w) for h, w in zip(report.HEADERS, widths)))
    for r in rows:
        print("  ".join(c.ljust(w) for c, w in zip(r.cells(), widths)))
    if args.out:
        report.write_csv(rows, args.out)
        print(f"report -> {args.out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
