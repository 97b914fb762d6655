"""Regenerate the golden fixtures in this directory (run from the repository root).

canonical_digests.json   SHA-256 of the canonical q/k/v bytes for a few cases,
                         pinning the seeded CPU generator (draw order, dtype,
                         stress transform) against silent changes.
attention_small.npz      one small case's canonical inputs and the float64
                         oracle output (stored as float32): a regression
                         fixture for the oracle and, on the GPU, for the
                         kernels.

The reference ships no golden vectors for this path (its tests pin only call
arguments), so these fixtures are produced by this repository's own oracle,
which tests/test_oracle.py pins independently (pure-loop definition, torch's
float64 scaled_dot_product_attention, closed forms, invariants).
"""

import hashlib
import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

import numpy as np  # noqa: E402

from fa_amd.problem.canonical import build_canonical  # noqa: E402
from fa_amd.problem.cases import CASES, Case  # noqa: E402
from oracle.attention import attention_f64  # noqa: E402

DIGEST_CASES = {
    "c0": CASES[0],
    "small": Case(1, 256, 2, 1),
    "small_stress": Case(1, 512, 12, 1, dist="stress"),
}
SMALL = DIGEST_CASES["small"]


def digests(case, seed=0):
    t = build_canonical(case, seed)
    return {n: hashlib.sha256(t[n].numpy().tobytes()).hexdigest() for n in ("q", "k", "v")}


def main():
    out = {name: {"case": case.name, "seed": 0, **digests(case)} for name, case in DIGEST_CASES.items()}
    (HERE / "canonical_digests.json").write_text(json.dumps(out, indent=1) + "\n")
    t = build_canonical(SMALL, 0)
    q, k, v = (t[n].numpy() for n in ("q", "k", "v"))
    np.savez_compressed(HERE / "attention_small.npz", q=q, k=k, v=v,
                        out=attention_f64(q, k, v).astype(np.float32))
    print("wrote", sorted(p.name for p in HERE.iterdir() if p.suffix in (".json", ".npz")))


if __name__ == "__main__":
    main()
