"""Golden fixtures: the canonical generator and the oracle against committed data."""

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from fa_amd.problem.canonical import build_canonical, stress_row_count
from fa_amd.problem.cases import CASES, Case
from oracle import attention as orc

GOLDEN = Path(__file__).resolve().parent / "golden"
CASES_BY_NAME = {c.name: c for c in (*CASES, Case(1, 256, 2, 1), Case(1, 512, 12, 1, dist="stress"))}


@pytest.mark.parametrize("key", sorted(json.loads((GOLDEN / "canonical_digests.json").read_text())))
def test_canonical_inputs_match_digests(key):
    entry = json.loads((GOLDEN / "canonical_digests.json").read_text())[key]
    t = build_canonical(CASES_BY_NAME[entry["case"]], entry["seed"])
    for n in ("q", "k", "v"):
        assert hashlib.sha256(t[n].numpy().tobytes()).hexdigest() == entry[n], n


def test_stress_transform_properties():
    case = Case(1, 512, 12, 1, dist="stress")
    t = build_canonical(case, 0)
    base = build_canonical(Case(1, 512, 12, 1), 0)
    # q and k are the same draws scaled by 3 (in FP16).
    assert np.array_equal(t["q"].numpy(), (base["q"] * 3).numpy())
    assert np.array_equal(t["k"].numpy(), (base["k"] * 3).numpy())
    # Exactly 5% of the v rows are the base rows times 8, the rest unchanged.
    v, v0 = t["v"].numpy().reshape(-1, 128), base["v"].numpy().reshape(-1, 128)
    scaled = ~np.all(v == v0, axis=1)
    assert scaled.sum() == stress_row_count(case) == 26
    assert np.array_equal(v[scaled], (v0[scaled].astype(np.float32) * 8).astype(np.float16))


def test_oracle_matches_golden_output():
    data = np.load(GOLDEN / "attention_small.npz")
    t = build_canonical(Case(1, 256, 2, 1), 0)
    for n in ("q", "k", "v"):
        assert np.array_equal(data[n], t[n].numpy())
    got = orc.attention_f64(data["q"], data["k"], data["v"])
    np.testing.assert_allclose(got, data["out"], rtol=2e-7, atol=1e-9)
