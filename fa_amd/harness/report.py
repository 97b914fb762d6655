"""Correctness checks and the per-case timing report across backends.

``check_backend`` runs one backend and the reference backend on the same
canonical inputs and compares the outputs the way the reference harness does
(``out.float()`` against ``ref.float()``: maximum absolute difference, and
``torch.testing.assert_close`` with atol = rtol = 1e-2 by default,
``core/runner.py:57-72`` there).

``run_case`` is one row group of the timing report: every selected backend is
prepared (libraries loaded) before the inputs are drawn, then bound to the
inputs and run once, timed (``timing.device_us``) and checked against the
reference. A backend that cannot be prepared or run is reported as skipped
instead of ending the report; a ``KernelNameError`` (a backend breaking the
kernel-naming rule) always propagates. Every backend must produce its output
from freshly allocated memory: the harness never clears device buffers for it.

The report columns are the reference's (``Case, Backend, Ref, Avg_us,
vs_ref, Check, MaxDiff``, ``core/bench.py:243-249`` there) plus QK/PV TFLOP/s
and the percentage of the dense FP16 MFMA peak.
"""

from __future__ import annotations

import csv
from dataclasses import dataclass

from fa_amd.harness import timing
from fa_amd.harness.contract import KernelNameError

# 256 CUs x 2.4 GHz x 4096 FP16 FLOP/clk/CU (dense MFMA).
PEAK_FP16_TFLOPS = 2516.6
HEADERS = ("Case", "Backend", "Ref", "Avg_us", "vs_ref", "Check", "MaxDiff", "TFLOPS", "PctPeak")


@dataclass(frozen=True)
class Tolerance:
    atol: float = 1e-2
    rtol: float = 1e-2


def compare(out, ref, tol: Tolerance):
    """(passed, max |out - ref|) over float32 copies of two tensors."""
    import torch

    a, b = out.float(), ref.float()
    worst = float((a - b).abs().max())
    try:
        torch.testing.assert_close(a, b, atol=tol.atol, rtol=tol.rtol)
        return True, worst
    except AssertionError:
        return False, worst


def check_backend(catalog, name, case, *, seed=0, tol=Tolerance(), device="cuda"):
    """Run backend ``name`` and the reference on one canonical input set.

    Returns ``(passed, max_abs_diff)``; the reference checked against itself
    passes with 0.
    """
    from fa_amd.problem.canonical import build_canonical

    entry = catalog.attention(name)
    ref = catalog.reference
    bind = catalog.prepare(name, case)
    ref_bind = None if entry.name == ref.name else catalog.prepare(ref.name, case)
    canonical = build_canonical(case, seed, device=device)
    out = bind(canonical)()
    if ref_bind is None:
        return True, 0.0
    return compare(out, ref_bind(canonical)(), tol)


def check_line(case, name, passed, diff, tol=Tolerance()) -> str:
    """The reference runner's one-line verdict."""
    status = "PASS" if passed else "FAIL"
    return (f"CHECK {case.name} backend={name} {status} max_abs_diff={diff:.5f} "
            f"(atol={tol.atol}, rtol={tol.rtol})")


@dataclass
class Row:
    case: str
    backend: str
    is_reference: bool
    avg_us: float | None = None
    vs_ref: float | None = None
    check: str = "skip"
    max_diff: float | None = None
    tflops: float | None = None

    def cells(self):
        def fmt(x, spec):
            return "N/A" if x is None else format(x, spec)

        pct = None if self.tflops is None else 100 * self.tflops / PEAK_FP16_TFLOPS
        return [self.case, self.backend, "ref" if self.is_reference else "",
                fmt(self.avg_us, ".2f"),
                "N/A" if self.vs_ref is None else f"{100 * self.vs_ref:.1f}%",
                self.check, fmt(self.max_diff, ".5f"), fmt(self.tflops, ".1f"),
                "N/A" if pct is None else f"{pct:.1f}%"]


def run_case(catalog, case, names, *, iters=20, seed=0, tol=Tolerance(), do_check=True,
             device="cuda", log=print):
    """Timing and check rows for ``names`` on one case (the reference is added)."""
    import torch

    from fa_amd.problem.canonical import build_canonical

    ref_name = catalog.reference.name
    order = [ref_name] + [n for n in names if n != ref_name]
    rows = {n: Row(case.name, n, n == ref_name) for n in order}

    binders = {}
    for n in order:
        try:
            binders[n] = catalog.prepare(n, case)
        except KernelNameError:
            raise
        except Exception as exc:                       # noqa: BLE001 -- reported, not fatal
            log(f"    [skip] {n}: cannot prepare: {exc}")
    canonical = build_canonical(case, seed, device=device)

    forwards = {}
    for n, bind in binders.items():
        try:
            forward = bind(canonical)
            forward()
            torch.cuda.synchronize()
            forwards[n] = forward
        except KernelNameError:
            raise
        except Exception as exc:                       # noqa: BLE001
            log(f"    [skip] {n}: first call failed: {exc}")

    for n, forward in forwards.items():
        us = timing.device_us(forward, iters=iters)
        rows[n].avg_us = us
        rows[n].tflops = case.flops / (us * 1e-6) / 1e12

    ref_us = rows[ref_name].avg_us
    for row in rows.values():
        if row.avg_us is not None and ref_us:
            row.vs_ref = row.avg_us / ref_us

    if do_check:
        ref_out = forwards[ref_name]().float().clone() if ref_name in forwards else None
        torch.cuda.synchronize()
        for n, forward in forwards.items():
            row = rows[n]
            if n == ref_name:
                row.check, row.max_diff = "ref", 0.0
            elif ref_out is None:
                row.check = "ERR"
            else:
                passed, row.max_diff = compare(forward(), ref_out, tol)
                row.check = "PASS" if passed else "FAIL"
        for n in order:
            if n not in forwards:
                rows[n].check = "ERR"
    return [rows[n] for n in order]


def write_csv(rows, path):
    with open(path, "w", newline="", encoding="utf-8") as f:
        w = csv.writer(f)
        w.writerow(HEADERS)
        w.writerows(r.cells() for r in rows)
