"""Seeded random configurations across every option of the forward at once.

Each case draws geometry (batch, GQA group, ragged Nq and Nk), accumulator,
causal mask, key-split count (none, automatic or explicit), tile selector,
strided (sequence-major) or contiguous layout, input distribution (N(0,1)
or the peaked stress form) and softmax scale, and checks O and lse against
the float64 oracle under the elementwise bounds of tests/test_gpu_parity.py.
Rows that see no key must give O = 0 and lse = -inf. The fixed lists of the
other GPU tests cover each option; this one covers their combinations.
"""

import random

import numpy as np
import pytest
import torch

from fa_amd.binding import AttentionConfig, Operator
from oracle import attention as orc

from test_gpu_parity import ATOL, LSE_ATOL, LSE_RTOL, P_ROUND, RTOL, say

pytestmark = pytest.mark.gpu

COUNT = 80


def draw(i, seed=20261202):
    rng = random.Random(seed * 1000 + i)
    hkv = rng.choice([1, 1, 2, 3])
    splits = rng.choice([None, None, 0, 1, 2, 3, 7, 40])
    return {
        "b": rng.choice([1, 2]), "hkv": hkv, "hq": hkv * rng.choice([1, 2, 4]),
        "nq": rng.choice([1, 2, 31, 64, 255, 256, 257, 300, 511, 600, 1000, 1500]),
        "nk": rng.choice([1, 5, 63, 64, 127, 128, 129, 500, 1000, 2047, 3000, 4100]),
        "acc": rng.choice(["fp32", "fp16"]),
        "causal": rng.choice(["none", "none", "top_left", "bottom_right"]),
        "splits": splits,
        "kernel": rng.choice([0, 0, 0, 1, 2, 3]) if splits is None else 0,
        "strided": rng.random() < 0.3,
        "sig": rng.choice([1.0, 1.0, 3.0]),
        "scale": rng.choice([None, None, 0.05, 0.2]),
    }


@pytest.fixture(scope="module")
def operators(library_path):
    cache = {}

    def get(cfg):
        if cfg not in cache:
            cache[cfg] = Operator(library_path, cfg)
        return cache[cfg]
    return get


@pytest.mark.parametrize("i", range(COUNT))
def test_random_configuration(operators, i):
    c = draw(i)
    say(f"case random config #{i}: {c}")
    g = torch.Generator().manual_seed(i * 7919 + 13)
    q = (torch.randn(c["b"], c["hq"], c["nq"], 128, generator=g) * c["sig"]).half()
    k = (torch.randn(c["b"], c["hkv"], c["nk"], 128, generator=g) * c["sig"]).half()
    v = torch.randn(c["b"], c["hkv"], c["nk"], 128, generator=g).half()
    if c["sig"] > 1:
        v[:, :, ::17] *= 8
    op = operators(AttentionConfig(acc=c["acc"], causal=c["causal"], splits=c["splits"],
                                   kernel=c["kernel"]))
    if c["strided"]:                   # [B, N, H, 128] memory viewed as [B, H, N, 128]
        dev = [t.transpose(1, 2).contiguous().cuda().transpose(1, 2) for t in (q, k, v)]
    else:
        dev = [t.cuda() for t in (q, k, v)]
    out, lse = op(*dev, scale=c["scale"], return_lse=True)
    torch.cuda.synchronize()
    out = out.float().cpu().numpy().astype(np.float64)
    lse = lse.cpu().numpy().astype(np.float64)
    acc, causal, scale = c["acc"], c["causal"], c["scale"]
    exact = orc.attention_f64(q, k, v, scale=scale, causal=causal)
    wabs = orc.attention_f64(q, k, v.abs(), scale=scale, causal=causal)
    exact_lse = orc.lse_f64(q, k, scale=scale, causal=causal)
    err = np.abs(out - exact)
    bound = ATOL[acc] + RTOL[acc] * np.abs(exact) + P_ROUND * (wabs + np.abs(exact))
    say(f"  max_abs={err.max():.3e} max_excess={(err - bound).max():.3e}")
    assert bool(np.all(np.isfinite(out))), "non-finite output"
    assert bool(np.all(err <= bound)), f"max abs error {err.max():.3e} exceeds the bound"
    none = np.isneginf(exact_lse)
    assert bool(np.all(out[none] == 0)) and bool(np.all(np.isneginf(lse[none]))), \
        "rows without keys must give O = 0 and lse = -inf"
    lerr = np.abs(lse[~none] - exact_lse[~none])
    assert bool(np.all(lerr <= LSE_ATOL + LSE_RTOL * np.abs(exact_lse[~none]))), \
        f"lse error {lerr.max():.3e}"


# Mid-size combinations: up to 9000 query rows and 70000 keys, up to 8 KV
# heads with groups up to 12, explicit tiles including the natural-V one,
# checked on sampled rows against the float64 oracle (the small cases above
# check every row).
MID_COUNT = 16


def draw_mid(i, seed=31):
    rng = random.Random(seed * 100000 + i)
    hkv = rng.choice([1, 1, 2, 4, 8])
    c = {
        "b": rng.choice([1, 2, 3]), "hkv": hkv, "hq": hkv * rng.choice([1, 2, 3, 6, 12]),
        "nq": rng.randint(1, 9000), "nk": rng.randint(1, 70000),
        "acc": rng.choice(["fp32", "fp16"]),
        "causal": rng.choice(["none", "none", "top_left", "bottom_right"]),
        "splits": rng.choice([None, None, None, 0, 2, 5]),
        "strided": rng.random() < 0.25,
        "sig": rng.choice([1.0, 1.0, 3.0]),
        "scale": rng.choice([None, None, 0.07]),
    }
    c["kernel"] = rng.choice([0, 0, 1, 2, 3, 4]) if c["splits"] is None else 0
    return c


@pytest.mark.parametrize("i", range(MID_COUNT))
def test_random_midsize_configuration_sampled_rows(operators, i):
    c = draw_mid(i)
    say(f"case random mid-size config #{i}: {c}")
    g = torch.Generator().manual_seed(i * 7919 + 31)
    q = (torch.randn(c["b"], c["hq"], c["nq"], 128, generator=g) * c["sig"]).half()
    k = (torch.randn(c["b"], c["hkv"], c["nk"], 128, generator=g) * c["sig"]).half()
    v = torch.randn(c["b"], c["hkv"], c["nk"], 128, generator=g).half()
    if c["sig"] > 1:
        v[:, :, ::19] *= 8
    op = operators(AttentionConfig(acc=c["acc"], causal=c["causal"], splits=c["splits"],
                                   kernel=c["kernel"]))
    if c["strided"]:
        dev = [t.transpose(1, 2).contiguous().cuda().transpose(1, 2) for t in (q, k, v)]
    else:
        dev = [t.cuda() for t in (q, k, v)]
    out, lse = op(*dev, scale=c["scale"], return_lse=True)
    torch.cuda.synchronize()
    rows = orc.sample_rows(q.shape, 48, seed=i)
    idx = torch.tensor(rows)
    got = out[idx[:, 0], idx[:, 1], idx[:, 2]].float().cpu().numpy().astype(np.float64)
    got_lse = lse[idx[:, 0], idx[:, 1], idx[:, 2]].cpu().numpy().astype(np.float64)
    del out, lse, dev
    acc, causal, scale = c["acc"], c["causal"], c["scale"]
    exact = orc.attention_rows_f64(q, k, v, rows, scale=scale, causal=causal)
    wabs = orc.attention_rows_f64(q, k, v.abs(), rows, scale=scale, causal=causal)
    exact_lse = orc.lse_rows_f64(q, k, rows, scale=scale, causal=causal)
    err = np.abs(got - exact)
    bound = ATOL[acc] + RTOL[acc] * np.abs(exact) + P_ROUND * (wabs + np.abs(exact))
    say(f"  max_abs={err.max():.3e} max_excess={(err - bound).max():.3e}")
    assert bool(np.all(np.isfinite(got))), "non-finite output"
    assert bool(np.all(err <= bound)), f"max abs error {err.max():.3e} exceeds the bound"
    none = np.isneginf(exact_lse)
    assert bool(np.all(got[none] == 0)) and bool(np.all(np.isneginf(got_lse[none])))
    lerr = np.abs(got_lse[~none] - exact_lse[~none])
    assert bool(np.all(lerr <= LSE_ATOL + LSE_RTOL * np.abs(exact_lse[~none]))), \
        f"lse error {lerr.max():.3e}"
