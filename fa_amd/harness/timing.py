"""Device time of backend forwards, and which backend a profiled kernel belongs to.

``device_us`` times one zero-argument forward with HIP events on torch's
current stream (the stream every backend here launches on): ``warmup``
untimed calls, then ``iters`` calls between two events, so the figure is the
device time of the whole forward -- every kernel it enqueues -- per call.
The reference reads the same quantity from its NPU profiler's kernel table
(3 warmup and 20 timed calls, ``core/profiler.py:28-85`` there).

``KernelOwners`` attributes kernel names from a ``rocprofv3 --kernel-trace``
run to backends, by the identity rule of the reference's plugin API
(``core/profiler.py:14-25``): a backend that declares its exact device
symbol owns only that symbol (and never claims a kernel by substring);
every other backend owns the kernels whose name contains its directory name
or its ``META.op_type``. A backend's exact symbol defaults to
``<directory>_kernel``. Explicit symbols are tried before any substring, so
``abc_kernel`` cannot be claimed by a backend called ``ab``.
``kernel_table`` applies it to a whole trace: each backend's mean device
kernel duration, the quantity the reference's profiler reports per backend
(``core/profiler.py:28-85``), with kernels no backend owns (for the HIP
backends, the prep kernel) listed apart.
"""

from __future__ import annotations

import csv
from collections import defaultdict


def device_us(forward, iters: int = 20, warmup: int = 3) -> float:
    """Average device microseconds per call of ``forward``."""
    import torch

    for _ in range(warmup):
        forward()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    begin = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    begin.record(stream)
    for _ in range(iters):
        forward()
    end.record(stream)
    torch.cuda.synchronize()
    return begin.elapsed_time(end) * 1e3 / iters


class KernelOwners:
    """Maps device kernel names to backend names."""

    def __init__(self, backends, op_types=None, symbols=None):
        self.backends = list(backends)
        self.op_types = dict(op_types or {})
        self.symbols = dict(symbols or {})      # backend -> exact declared symbol

    def owner(self, kernel_name: str):
        exact = {self.symbols.get(b, f"{b}_kernel"): b for b in self.backends}
        if kernel_name in exact:
            return exact[kernel_name]
        for b in self.backends:
            if b in self.symbols:
                continue                          # declared symbols match exactly or not at all
            needles = [b] + ([self.op_types[b]] if self.op_types.get(b) else [])
            if any(n in kernel_name for n in needles):
                return b
        return None

    def average_us(self, trace_csv) -> dict:
        """Per-backend mean kernel duration (us) in a rocprofv3 kernel-trace CSV."""
        durations = defaultdict(list)
        with open(trace_csv, newline="", encoding="utf-8") as f:
            for rec in csv.DictReader(f):
                b = self.owner(rec.get("Kernel_Name", ""))
                if b is not None:
                    ns = int(rec["End_Timestamp"]) - int(rec["Start_Timestamp"])
                    durations[b].append(ns / 1e3)
        return {b: (sum(durations[b]) / len(durations[b]) if durations[b] else None)
                for b in self.backends}


def kernel_table(trace_dir, owners: KernelOwners, skip: int = 0):
    """Per-backend kernel durations of a rocprofv3 kernel trace.

    Reads every dispatch under ``trace_dir`` (CSV or rocpd output, via
    ``fa_amd.measure.kernel_stats``), drops the first ``skip`` dispatches of
    every kernel (warmup calls), and returns ``(per_backend, unowned)``:
    ``per_backend[b] = {"dispatches": n, "mean_us": ..., "kernels": [names]}``
    (None for a backend with no dispatch) and ``unowned[name] = (n, mean_us)``.
    """
    from fa_amd.measure import kernel_stats

    stats = kernel_stats.skip_first(kernel_stats.collect(trace_dir), skip)
    per = {b: [] for b in owners.backends}
    names = {b: [] for b in owners.backends}
    unowned = {}
    for name, durs in stats.items():
        b = owners.owner(name)
        if b is None:
            unowned[name] = (len(durs), sum(durs) / len(durs) / 1e3)
        else:
            per[b].extend(durs)
            names[b].append(name)
    table = {b: ({"dispatches": len(d), "mean_us": sum(d) / len(d) / 1e3, "kernels": names[b]}
                 if d else None) for b, d in per.items()}
    return table, unowned


def render_kernel_table(table, unowned, max_unowned=5):
    """Text table: one line per backend, then the ``max_unowned`` unowned
    kernels with the most device time and a line summing the rest."""
    lines = [f"{'Backend':<18} {'Dispatches':>10} {'Kernel_us':>14}  Kernels"]
    for b, row in table.items():
        if row is None:
            lines.append(f"{b:<18} {0:>10} {'N/A':>14}  (no kernel of this backend in the trace)")
        else:
            lines.append(f"{b:<18} {row['dispatches']:>10} {row['mean_us']:>14,.2f}  "
                         + "; ".join(row["kernels"]))
    ranked = sorted(unowned.items(), key=lambda kv: -kv[1][0] * kv[1][1])
    for name, (n, us) in ranked[:max_unowned]:
        lines.append(f"{'(unowned)':<18} {n:>10} {us:>14,.2f}  {name}")
    rest = ranked[max_unowned:]
    if rest:
        lines.append(f"{'(unowned)':<18} {sum(n for _, (n, _) in rest):>10} {'':>14}  "
                     f"... {len(rest)} more kernels, {sum(n * us for _, (n, us) in rest):,.0f} us in all")
    return "\n".join(lines)
