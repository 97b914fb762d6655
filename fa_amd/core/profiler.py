"""Device-time profiling of backends on the current GPU stream.

``profile_case_us`` mirrors the reference's ``core/profiler.py:28-85``: warm
every backend up, then time ``iters`` calls of each and return the average
per-call device time in microseconds. The reference reads a torch_npu
profiler's kernel table; here every backend's calls are bracketed by HIP
events on torch's current stream, the stream all backends launch on, so the
figure is the device time of the whole forward (all kernels it enqueues).

``kernel_times_us`` parses a ``rocprofv3 --kernel-trace`` CSV into the same
per-backend averages, attributing each kernel by ``_match_backend``: exact
symbols first, then the backend directory name or ``META.op_type`` as a
substring (reference ``core/profiler.py:14-25``).
"""

import csv


def _match_backend(name, backend_names, op_types, kernel_names):
    """Match explicit symbols exactly; only the others use substring filters."""
    for n in backend_names:
        if name == kernel_names.get(n, f"{n}_kernel"):
            return n
    for n in backend_names:
        if n in kernel_names:
            continue
        op = op_types.get(n, "")
        if (n in name) or (op and op in name):
            return n
    return None


def profile_case_us(calls, backend_names, iters=20, warmup=3):
    """Average device microseconds per call for each backend in ``calls``.

    ``calls`` maps backend name -> zero-argument callable; names missing from
    it map to None in the result.
    """
    import torch

    times = {}
    for n in backend_names:
        if n not in calls:
            times[n] = None
            continue
        for _ in range(warmup):
            calls[n]()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(iters):
            calls[n]()
        end.record(stream)
        torch.cuda.synchronize()
        times[n] = start.elapsed_time(end) * 1e3 / iters
    return times


def kernel_times_us(trace_csv, backend_names, op_types=None, kernel_names=None):
    """Per-backend average kernel duration (us) from a rocprofv3 kernel-trace CSV."""
    op_types = op_types or {}
    kernel_names = kernel_names or {}
    by_backend = {}
    with open(trace_csv, newline="", encoding="utf-8") as f:
        for row in csv.DictReader(f):
            n = _match_backend(row.get("Kernel_Name", ""), backend_names, op_types, kernel_names)
            if n is None:
                continue
            dur = (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3
            by_backend.setdefault(n, []).append(dur)
    return {n: (sum(v) / len(v) if v else None)
            for n in backend_names for v in [by_backend.get(n, [])]}
