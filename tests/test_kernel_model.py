"""The CPU model of the kernel's rounding (tests/kernel_model.py), pinned on the CPU.

With rounding off, the model's blocked computation -- key blocks, the lazy
running max with TAU = 8 or 0, the alpha rescales, the FP16-accumulator's
per-block merge order -- must reproduce the float64 oracle to float64
precision, so a wrong recurrence (a misplaced alpha, a merge applied to the
wrong block, a row sum over the wrong weights) fails here before the model is
trusted against the kernel. With rounding on, the model must differ from the
oracle by no more than the bound that FP16-rounded P allows, and must differ
at all (the roundings are really applied).
"""

import numpy as np
import pytest
import torch

import kernel_model as km
from oracle import attention as orc


def draw(b, hq, hkv, nq, nk, sig, seed, spikes=False):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(b, hq, nq, 128, generator=g) * sig).half()
    k = (torch.randn(b, hkv, nk, 128, generator=g) * sig).half()
    v = torch.randn(b, hkv, nk, 128, generator=g)
    if spikes:                                  # the stress configuration's x8 value rows
        rows = torch.randperm(nk, generator=g)[: max(1, nk // 20)]
        v[:, :, rows] *= 8
    return q, k, v.half()


SHAPES = [(1, 4, 2, 40, 300, 1.0, False), (2, 6, 3, 17, 1000, 3.0, True),
          (1, 2, 1, 33, 4096, 3.0, True), (1, 2, 1, 20, 129, 1.0, False)]


@pytest.mark.parametrize("acc,block", [("fp32", 128), ("fp16", 64), ("fp32", 64), ("fp16", 128)])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[3]}x{s[4]}_sig{s[5]}")
def test_model_without_rounding_is_the_oracle(acc, block, shape):
    b, hq, hkv, nq, nk, sig, spikes = shape
    q, k, v = draw(b, hq, hkv, nq, nk, sig, seed=nk + nq, spikes=spikes)
    rows = orc.sample_rows(q.shape, 24, seed=3)
    out, extra = km.model_rows(q, k, v, rows, acc=acc, block=block, rounding=False)
    exact = orc.attention_rows_f64(q, k, v, rows)
    assert np.abs(out - exact).max() <= 1e-9 * max(1.0, np.abs(exact).max())
    assert not extra.any()


@pytest.mark.parametrize("acc", ["fp32", "fp16"])
def test_model_with_rounding_stays_within_the_p_rounding_bound(acc):
    q, k, v = draw(1, 4, 1, 64, 2048, 3.0, seed=5, spikes=True)
    rows = orc.sample_rows(q.shape, 64, seed=4)
    block = 128 if acc == "fp32" else 64
    out, _ = km.model_rows(q, k, v, rows, acc=acc, block=block)
    exact = orc.attention_rows_f64(q, k, v, rows)
    wabs = orc.attention_rows_f64(q, k, v.abs(), rows)
    err = np.abs(out - exact)
    assert err.max() > 0                               # roundings are applied
    rtol = 2.0 ** -10 if acc == "fp32" else 2.0 ** -6  # output ulp; FP16 merges of |O| ~ 30
    assert np.all(err <= 2e-3 + rtol * np.abs(exact) + 2.0 ** -11 * (wabs + np.abs(exact)))


def test_scores_follow_the_mfma_k_steps():
    g = torch.Generator().manual_seed(1)
    q = (torch.randn(3, 128, generator=g) * 3).half().numpy()
    k = (torch.randn(50, 128, generator=g) * 3).half().numpy()
    s = km.scores_mfma(q, k)
    exact = q.astype(np.float64) @ k.astype(np.float64).T
    mag = np.abs(q.astype(np.float64)) @ np.abs(k.astype(np.float64)).T
    assert s.dtype == np.float32
    assert np.all(np.abs(s - exact) <= 8 * 2.0 ** -24 * mag)
    # Eight FP32 roundings in k-step order, not one rounding of the exact sum.
    assert np.any(s != exact.astype(np.float32))


def test_midpoint_detection_and_tolerance():
    one_ulp = 2.0 ** -10                       # FP16 ulp in [1, 2)
    mid = 1.0 + one_ulp / 2
    # Exactly on a midpoint is an exact value computed identically (not
    # ambiguous); just beside it, it is; a quarter ulp away it is not.
    assert km._near_midpoint(np.array([mid, mid * (1 + 2 ** -20), 1.0 + one_ulp / 4])).tolist() \
        == [False, True, False]
    assert km._ulp16(np.array([1.0, 3.0, 0.25]))[1] == 2.0 ** -9
    tol = km.tolerance(np.array([1.5]), np.array([0.0]))
    assert km.tolerance(np.array([1.5]), np.array([0.0]), acc="fp16")[0] > tol[0]
    assert tol[0] == pytest.approx(2.0 ** -10 + 1.5e-4 + km.ABS_FLOOR)
