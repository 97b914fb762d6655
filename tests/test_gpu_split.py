"""GPU parity of the key-split forward (fa_fwd_split) against the CPU oracle.

The split forward runs every (query tile, key-range part) as its own work
item and merges the parts' (O, lse) pairs in a second kernel, so its output
differs from the one-pass forward's only by FP32 summation order (and, for
the FP16 accumulator, by where the 512-key packets start). It is held to the
same elementwise bounds against the float64 oracle as the one-pass forward
(tests/test_gpu_parity.py), and a count of 1 must be the one-pass forward bit
for bit. Every case prints its name before its GPU work.
"""

import numpy as np
import pytest
import torch

from fa_amd.binding import AttentionConfig, Operator
from oracle import attention as orc

from test_gpu_parity import check, check_lse, say

pytestmark = pytest.mark.gpu


def make(b, hq, hkv, nq, nk, seed, sig=1.0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(b, hq, nq, 128, generator=g) * sig).half()
    k = (torch.randn(b, hkv, nk, 128, generator=g) * sig).half()
    v = torch.randn(b, hkv, nk, 128, generator=g).half()
    if sig > 1:
        v[:, :, ::23] *= 8
    return q, k, v


# (B, Hq, Hkv, Nq, Nk, causal, splits); splits 0 = the library's choice.
SHAPES = [
    (1, 12, 1, 256, 8192, "none", 0),
    (1, 12, 1, 256, 8192, "none", 5),
    (1, 4, 1, 1, 4096, "none", 0),           # one query row per head
    (2, 4, 2, 300, 3000, "none", 3),          # ragged query and key tails
    (1, 2, 2, 70, 1000, "none", 100),         # clamped to the 8 key blocks
    (1, 4, 1, 1000, 1000, "top_left", 4),     # later parts of early tiles are empty
    (1, 2, 2, 200, 777, "bottom_right", 3),
    (1, 2, 1, 700, 300, "bottom_right", 2),   # rows 0..399 see no key at all
    (1, 6, 3, 512, 5000, "top_left", 0),
]


@pytest.mark.parametrize("acc", ["fp32", "fp16"])
@pytest.mark.parametrize("b,hq,hkv,nq,nk,causal,splits", SHAPES)
def test_split_vs_f64(library_path, b, hq, hkv, nq, nk, causal, splits, acc):
    say(f"case split B{b} Hq{hq} Hkv{hkv} nq={nq} nk={nk} causal={causal} splits={splits} acc={acc}")
    q, k, v = make(b, hq, hkv, nq, nk, seed=nq * 31 + nk + splits)
    op = Operator(library_path, AttentionConfig(acc=acc, causal=causal, splits=splits))
    used = op.split_count(q.shape, k.shape)
    say(f"  parts per tile: {used}")
    if splits:
        assert used == min(splits, -(-nk // 128))
    out, lse = op(q.cuda(), k.cuda(), v.cuda(), return_lse=True)
    torch.cuda.synchronize()
    out = out.float().cpu().numpy()
    check(out, orc.attention_f64(q, k, v, causal=causal), acc, "split",
          orc.attention_f64(q, k, v.abs(), causal=causal))
    exact_lse = orc.lse_f64(q, k, causal=causal)
    check_lse(lse.cpu().numpy(), exact_lse, "split")
    empty = np.isneginf(exact_lse)
    assert bool(np.all(out[empty] == 0)), "rows without keys must be exactly zero"


@pytest.mark.parametrize("acc", ["fp32", "fp16"])
def test_split_stress(library_path, acc):
    """Peaked rows (q, k ~ 3 N(0,1), every 23rd value row x8), 7 parts."""
    say(f"case split stress nq=300 nk=4000 acc={acc}")
    q, k, v = make(1, 6, 2, 300, 4000, seed=11, sig=3.0)
    op = Operator(library_path, AttentionConfig(acc=acc, splits=7))
    out, lse = op(q.cuda(), k.cuda(), v.cuda(), return_lse=True)
    torch.cuda.synchronize()
    check(out.float().cpu().numpy(), orc.attention_f64(q, k, v), acc, "split stress",
          orc.attention_f64(q, k, v.abs()))
    check_lse(lse.cpu().numpy(), orc.lse_f64(q, k), "split stress")


@pytest.mark.parametrize("causal", ["none", "top_left"])
def test_one_part_is_the_one_pass_forward(library_path, causal):
    """splits = 1 runs fa_fwd_lse(): output and lse equal bit for bit."""
    say(f"case split=1 equals fa_fwd_lse causal={causal}")
    q, k, v = make(1, 4, 1, 600, 2000, seed=5)
    dev = [t.cuda() for t in (q, k, v)]
    for acc in ("fp32", "fp16"):
        a, la = Operator(library_path, AttentionConfig(acc=acc, causal=causal))(*dev, return_lse=True)
        a, la = a.clone(), la.clone()
        b, lb = Operator(library_path, AttentionConfig(acc=acc, causal=causal, splits=1))(
            *dev, return_lse=True)
        torch.cuda.synchronize()
        assert bool(torch.equal(a, b)) and bool(torch.equal(la, lb)), acc


def test_split_repeatable_and_strided(library_path):
    """Two calls give the same bits (the work queue hands parts to CUs in any
    order, but each part's arithmetic and the merge order are fixed); a
    sequence-major view gives the bits of its contiguous copy."""
    say("case split repeat + strided B1 Hq8 Hkv2 nq=384 nk=6000 splits=6")
    g = torch.Generator().manual_seed(9)
    qs = torch.randn(1, 384, 8, 128, generator=g, dtype=torch.float16).cuda()
    ks = torch.randn(1, 6000, 2, 128, generator=g, dtype=torch.float16).cuda()
    vs = torch.randn(1, 6000, 2, 128, generator=g, dtype=torch.float16).cuda()
    q, k, v = (t.transpose(1, 2) for t in (qs, ks, vs))
    for acc in ("fp32", "fp16"):
        op = Operator(library_path, AttentionConfig(acc=acc, splits=6))
        first, l1 = (t.clone() for t in op(q, k, v, return_lse=True))
        again, l2 = (t.clone() for t in op(q, k, v, return_lse=True))
        cont, l3 = op(q.contiguous(), k.contiguous(), v.contiguous(), return_lse=True)
        torch.cuda.synchronize()
        assert bool(torch.equal(first, again)) and bool(torch.equal(l1, l2)), acc
        assert bool(torch.equal(first, cont)) and bool(torch.equal(l1, l3)), acc
        check(first.float().cpu().numpy(), orc.attention_f64(q.cpu(), k.cpu(), v.cpu()), acc,
              "split strided")


def test_split_long_keys_sampled_rows(library_path):
    """12 query tiles against 131072 keys (the shape the split exists for):
    the library's own count, sampled rows against the float64 oracle, and
    the split forward faster than the one-pass forward."""
    nq, nk = 256, 131072
    say(f"case split long B1 Hq12 nq={nq} nk={nk}")
    q, k, v = make(1, 12, 1, nq, nk, seed=21)
    dev = [t.cuda() for t in (q, k, v)]
    rows = orc.sample_rows(q.shape, 48, seed=4)
    for acc in ("fp32", "fp16"):
        split = Operator(library_path, AttentionConfig(acc=acc, splits=0))
        assert split.split_count(q.shape, k.shape) > 1
        one = Operator(library_path, AttentionConfig(acc=acc))
        times = {}
        for name, op in (("one-pass", one), ("split", split)):
            op(*dev)
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            for _ in range(3):
                out = op(*dev)
            end.record()
            torch.cuda.synchronize()
            times[name] = start.elapsed_time(end) / 3
        say(f"  {acc}: one-pass {times['one-pass']:.3f} ms, split "
            f"({split.split_count(q.shape, k.shape)} parts) {times['split']:.3f} ms")
        got = out.float().cpu().numpy()[tuple(np.array(rows).T)]
        check(got, orc.attention_rows_f64(q, k, v, rows), acc, "split long")
        assert times["split"] < 0.5 * times["one-pass"], times


@pytest.mark.parametrize("acc", ["fp32", "fp16"])
@pytest.mark.parametrize("causal", ["none", "bottom_right"])
def test_split_million_keys_sampled_rows(library_path, causal, acc):
    """A million ragged keys (the parts' buffer offsets and ranges near their
    32-bit limits) against 512 query rows of 4 heads (8 tiles, which the
    automatic count cuts into 32 parts each), sampled rows against the
    float64 oracle."""
    nq, nk = 512, 1_048_573
    say(f"case split million keys nq={nq} nk={nk} causal={causal} acc={acc}: generating inputs")
    q, k, v = make(1, 4, 1, nq, nk, seed=nk % 1000 + nq)
    op = Operator(library_path, AttentionConfig(acc=acc, causal=causal, splits=0))
    say(f"  parts per tile: {op.split_count(q.shape, k.shape)}")
    out, lse = op(q.cuda(), k.cuda(), v.cuda(), return_lse=True)
    torch.cuda.synchronize()
    rows = orc.sample_rows(q.shape, 24, seed=nq + nk)
    idx = torch.tensor(rows)
    got = out[idx[:, 0], idx[:, 1], idx[:, 2]].float().cpu().numpy()
    check(got, orc.attention_rows_f64(q, k, v, rows, causal=causal), acc, "split million keys",
          orc.attention_rows_f64(q, k, v.abs(), rows, causal=causal))
    check_lse(lse[idx[:, 0], idx[:, 1], idx[:, 2]].cpu().numpy(),
              orc.lse_rows_f64(q, k, rows, causal=causal), "split million keys")


def test_split_graph_capture_replays(library_path):
    """fa_fwd_split captured in a HIP graph (three kernels, no memset): every
    replay, with eager work and synchronisation in between and the inputs
    changed in place, equals the eager split forward for the current inputs."""
    say("case split graph capture B1 Hq12 nq=256 nk=8192 splits=6")
    g = torch.Generator().manual_seed(23)
    q = torch.randn(1, 12, 256, 128, generator=g, dtype=torch.float16).cuda()
    k = torch.randn(1, 1, 8192, 128, generator=g, dtype=torch.float16).cuda()
    v = torch.randn(1, 1, 8192, 128, generator=g, dtype=torch.float16).cuda()
    op = Operator(library_path, AttentionConfig(splits=6))
    op(q, k, v, return_lse=True)                  # allocates the cached outputs and workspace
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            out, lse = op(q, k, v, return_lse=True)
    torch.cuda.synchronize()
    eager = Operator(library_path, AttentionConfig(splits=6))
    for rep in range(4):
        q.copy_(torch.randn(q.shape, generator=g, dtype=torch.float16).cuda())
        v.mul_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want, want_lse = eager(q, k, v, return_lse=True)
        torch.cuda.synchronize()
        assert bool(torch.equal(out, want)) and bool(torch.equal(lse, want_lse)), rep
