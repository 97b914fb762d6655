"""The kernel against the CPU model of its own rounding (tests/kernel_model.py).

The stress configuration (c4: q, k ~ 3 N(0,1), 5% of the value rows x8)
exceeds the north-star's literal absolute bars on a few rows: peaked softmax
rows whose dominant keys carry x8 value rows. These tests show where that
excess comes from. The model repeats every rounding the kernel performs
(FP32 scores in MFMA k-step order, the lazy running max, FP16-rounded P,
the row sum, the FP32 or FP16 O accumulation and its merges, the final FP16
output); the kernel must match it to within one or a few output ulps plus the
effect of the P roundings the model cannot decide (P within a few FP32 ulps
of an FP16 rounding midpoint), while its distance from the float64 oracle --
the part every kernel that feeds FP16 P to the matrix cores must have -- is
carried by the model itself. Rows are the full small stress shapes, and at
c4 the worst rows of the full-size output (against the FP32 formula on the
GPU) plus a random sample.
"""

import numpy as np
import pytest
import torch

import kernel_model as km
from fa_amd.binding import AttentionConfig, Operator
from fa_amd.problem.canonical import build_canonical
from fa_amd.problem.cases import CASES
from oracle import attention as orc

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


def block_of(op, q, k):
    name = op.kernel_name(q.shape, k.shape)          # pp_n{keys}_r{ring}
    return int(name.split("_")[1][1:])


def compare(what, acc, got, model, extra, exact):
    tol = km.tolerance(model, extra, acc)
    d_km = np.abs(got - model)
    d_me = np.abs(model - exact)
    d_ke = np.abs(got - exact)
    ulp = km._ulp16(np.abs(model))
    plain = extra < 0.25 * ulp              # elements no undecidable P rounding can move
    exact_frac = float(np.mean(d_km == 0))
    say(f"  {what} acc={acc}: |kernel-model| max {d_km.max():.3e} "
        f"({(d_km / ulp).max():.2f} output ulps; {100 * exact_frac:.2f}% of elements bit-exact; "
        f"on the {100 * np.mean(plain):.1f}% no undecidable P rounding reaches: "
        f"{(d_km[plain] / ulp[plain]).max() if plain.any() else 0:.2f} ulps); "
        f"|model-f64| max {d_me.max():.3e}; |kernel-f64| max {d_ke.max():.3e} "
        f"({(d_ke / ulp).max():.1f} output ulps)")
    assert np.all(np.isfinite(got))
    worst = float((d_km - tol).max())
    assert np.all(d_km <= tol), f"{what}: kernel departs from the rounding model by {worst:.3e} beyond the bound"
    assert exact_frac >= 0.99
    return d_km.max(), d_me.max(), d_ke.max()


def draw_stress(b, hq, hkv, nq, nk, seed):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(b, hq, nq, 128, generator=g) * 3).half()
    k = (torch.randn(b, hkv, nk, 128, generator=g) * 3).half()
    v = torch.randn(b, hkv, nk, 128, generator=g)
    rows = torch.randperm(b * hkv * nk, generator=g)[: (b * hkv * nk) // 20]
    v.view(-1, 128)[rows] *= 8
    return q, k, v.half()


@pytest.mark.parametrize("acc", ["fp32", "fp16"])
@pytest.mark.parametrize("shape", [(1, 4, 1, 512, 2048), (2, 6, 2, 300, 1000)],
                         ids=["512x2048", "ragged300x1000"])
def test_stress_shapes_every_row_match_the_model(library_path, acc, shape):
    b, hq, hkv, nq, nk = shape
    say(f"case model stress {shape} acc={acc}")
    q, k, v = draw_stress(b, hq, hkv, nq, nk, seed=nq + nk)
    op = Operator(library_path, AttentionConfig(acc=acc))
    out = op(q.cuda(), k.cuda(), v.cuda()).float().cpu().numpy()
    torch.cuda.synchronize()
    rows = [(bi, h, i) for bi in range(b) for h in range(hq) for i in range(nq)]
    model, extra = km.model_rows(q, k, v, rows, acc=acc, block=block_of(op, q, k))
    exact = orc.attention_rows_f64(q, k, v, rows)
    got = np.stack([out[bi, h, i] for bi, h, i in rows])
    compare(f"stress {shape}", acc, got, model, extra, exact)


@pytest.mark.parametrize("acc", ["fp32", "fp16"])
def test_c4_worst_rows_match_the_model(library_path, acc):
    from fa_amd.backends.torch_ref import backend as torch_ref

    case = CASES[4]
    say(f"case model c4 {case.name} acc={acc}: inputs")
    cpu = build_canonical(case)
    dev = {n: t.cuda() for n, t in cpu.items()}
    op = Operator(library_path, AttentionConfig(acc=acc))
    say(f"case model c4 acc={acc}: kernel and FP32 formula on the GPU")
    out = op(dev["q"], dev["k"], dev["v"]).clone()
    ref = torch_ref.attention(dev["q"], dev["k"], dev["v"], case.scale)
    torch.cuda.synchronize()
    diff = (out.float() - ref.float()).abs()
    row_err = diff.amax(dim=3).cpu().numpy()                                   # [B, Hq, Nq]
    # The reference harness's own check (core/bench.py:139, atol = rtol = 1e-2),
    # row by row: the model of the reference kernels' roundings fails it on
    # about 4 % of c4's rows (tests/test_reference_model.py); this kernel on
    # at most one row in ten thousand.
    failing = int((diff > 1e-2 + 1e-2 * ref.float().abs()).any(dim=3).sum())
    say(f"  rows failing the reference harness's check: {failing} of {row_err.size}")
    assert failing <= row_err.size // 10000
    del ref, diff
    worst = np.argsort(row_err.ravel())[-24:]
    shape = row_err.shape
    rows = {tuple(int(x) for x in np.unravel_index(f, shape)) for f in worst}
    rows |= set(orc.sample_rows(cpu["q"].shape, 24, seed=44))
    rows = sorted(rows)
    say(f"  {len(rows)} rows (24 worst against the FP32 formula: {row_err.max():.3e} max); model on CPU")
    model, extra = km.model_rows(cpu["q"], cpu["k"], cpu["v"], rows, acc=acc,
                                 block=block_of(op, dev["q"], dev["k"]))
    exact = orc.attention_rows_f64(cpu["q"], cpu["k"], cpu["v"], rows)
    idx = torch.tensor(rows)
    got = out[idx[:, 0], idx[:, 1], idx[:, 2]].float().cpu().numpy()
    d_km, d_me, d_ke = compare("c4 worst + sampled rows", acc, got, model, extra, exact)
    # The excess over the float64 result is the model's own: the modelled
    # roundings alone reproduce most of the kernel's distance from it.
    assert d_me >= 0.5 * d_ke
    del dev, out
    torch.cuda.empty_cache()
