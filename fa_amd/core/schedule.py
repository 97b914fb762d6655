"""Execution scheduling primitives (reference ``core/schedule.py:16-22``).

``parallel_compile`` runs compile tasks on a CPU process pool (no GPU is
touched). The reference's multi-card fan-out has no counterpart: this build
targets one GPU, and a case runs in the calling process.
"""

import os
from concurrent.futures import ProcessPoolExecutor


def parallel_compile(items, compile_one, workers=None):
    """Run ``compile_one(item)`` for every item on a CPU process pool."""
    if not items:
        return []
    workers = workers or min(len(items), os.cpu_count() or 1)
    with ProcessPoolExecutor(max_workers=workers) as pool:
        return list(pool.map(compile_one, items))
