"""Single (backend x case) execution, run as its own process.

Modes (reference ``core/runner.py:1-72``):
  compile : build the backend through its driver; touches no GPU.
  check   : run the backend and the reference backend once on the canonical
            inputs and compare: prints
            ``CHECK <case> backend=<name> PASS|FAIL max_abs_diff=<d> (atol=.., rtol=..)``.
A fresh process gives every check freshly allocated device memory, so a
backend that read uninitialised workspace could not pass on leftovers.

Heavy imports stay inside main() so the compile path stays light.
"""

import argparse
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))


def _parse_args(argv=None):
    p = argparse.ArgumentParser(description="single runner")
    p.add_argument("--backend", required=True)
    p.add_argument("--case-index", type=int, required=True)
    p.add_argument("--mode", choices=("compile", "check"), default="check")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--atol", type=float, default=1e-2)
    p.add_argument("--rtol", type=float, default=1e-2)
    return p.parse_args(argv)


def main(argv=None):
    args = _parse_args(argv)

    from fa_amd.core import registry
    from fa_amd.problem.cases import CASES

    case = CASES[args.case_index]
    spec = registry.get(args.backend)
    registry.require_attention(spec)
    meta = spec.META
    driver = registry.driver_for(meta)

    if args.mode == "compile":
        driver.compile(spec, case)
        print(f"COMPILE {args.backend} {case.name} done")
        return 0

    import torch

    from fa_amd.problem.canonical import build_canonical

    bind = registry.prepare_call(spec, case)
    if not meta.is_reference:
        _, ref_spec = registry.get_reference()
        ref_bind = registry.prepare_call(ref_spec, case)
    canonical = build_canonical(case, args.seed, device="cuda")
    out = bind(canonical)().float()

    if meta.is_reference:
        print(f"CHECK {case.name} backend={args.backend} PASS max_abs_diff=0.00000 (self)")
        return 0

    ref_out = ref_bind(canonical)().float()
    torch.cuda.synchronize()
    max_diff = (out - ref_out).abs().max().item()
    try:
        torch.testing.assert_close(out, ref_out, atol=args.atol, rtol=args.rtol)
        status = "PASS"
    except AssertionError:
        status = "FAIL"
    print(f"CHECK {case.name} backend={args.backend} {status} "
          f"max_abs_diff={max_diff:.5f} (atol={args.atol}, rtol={args.rtol})")
    return 0 if status == "PASS" else 1


if __name__ == "__main__":
    sys.exit(main())
