"""Packed tiles on the GPU: grouped-query attention with few query rows.

When the query heads that share a KV head have fewer query rows than a tile
holds, the library packs the group's rows position by position into one
tile instead of giving each head a tile of its own (the rule is
``fa_amd.binding.query_tiles``). Each row's computation (its keys, its block
order, its roundings) does not depend on which tile it sits in, so a packed
row must equal the same row computed unpacked bit for bit. The unpacked
reference here is the same problem with 256 (or 512) query rows per head,
whose first rows are the packed problem's rows: that layout is never packed.
Top-left causal masks keep every row's key limit between the two; the
bottom-right mask and decode shapes (one query row, long keys, the key-split
forward) are checked against the float64 oracle. Every case prints its name
before its GPU work.
"""

import numpy as np
import pytest
import torch

from fa_amd import binding
from fa_amd.binding import AttentionConfig, Operator
from oracle import attention as orc

from test_gpu_parity import check, check_lse, say

pytestmark = pytest.mark.gpu


def draw(b, hq, hkv, nq, nk, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, nq, 128, generator=g).half()
    k = torch.randn(b, hkv, nk, 128, generator=g).half()
    v = torch.randn(b, hkv, nk, 128, generator=g).half()
    return q, k, v


def plain_tiles(b, hq, nq):
    return b * hq * -(-nq // 256)


# (Hq, Hkv, Nq, Nk): groups of 12, 4 and 2 query heads; Nq from one row to a
# ragged 300 (two tiles per head unpacked, fifteen per group packed).
PACKED = [
    (12, 1, 1, 1000), (12, 1, 7, 2048), (12, 1, 21, 1000), (12, 1, 22, 3000), (12, 1, 100, 777),
    (12, 1, 300, 1500), (8, 2, 5, 1000), (8, 2, 64, 2048), (8, 2, 63, 513), (6, 3, 128, 1000),
    (6, 3, 1, 4096),
]


@pytest.mark.parametrize("acc", ["fp32", "fp16"])
@pytest.mark.parametrize("causal", ["none", "top_left"])
@pytest.mark.parametrize("hq,hkv,nq,nk", PACKED, ids=lambda x: str(x))
def test_packed_rows_equal_unpacked_rows(library_path, hq, hkv, nq, nk, causal, acc):
    b = 2
    big = 256 if nq <= 256 else 512
    assert binding.query_tiles(b, hq, hkv, nq) < plain_tiles(b, hq, nq), "the case must pack"
    assert binding.query_tiles(b, hq, hkv, big) == plain_tiles(b, hq, big), "the reference must not"
    say(f"case packed B{b} Hq{hq} Hkv{hkv} nq={nq} (tiles {binding.query_tiles(b, hq, hkv, nq)} "
        f"instead of {plain_tiles(b, hq, nq)}) nk={nk} causal={causal} acc={acc}")
    qbig, k, v = draw(b, hq, hkv, big, nk, seed=hq * 1000 + nq * 7 + nk)
    qbig, k, v = qbig.cuda(), k.cuda(), v.cuda()
    q = qbig[:, :, :nq].contiguous()
    op = Operator(library_path, AttentionConfig(acc=acc, causal=causal))
    o_big, l_big = (t.clone() for t in op(qbig, k, v, return_lse=True))
    o, lse = op(q, k, v, return_lse=True)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all()
    diff = (o.float() - o_big[:, :, :nq].float()).abs().max().item()
    assert torch.equal(o, o_big[:, :, :nq]), f"max |diff| {diff:.3e}"
    assert torch.equal(lse, l_big[:, :, :nq])


# (B, Hq, Hkv, Nq, Nk, causal, splits): decode and speculative-decode shapes
# through the one-pass and the key-split forward (None: one pass; 0: the
# library's count).
DECODE = [
    (1, 12, 1, 1, 65536, "none", 0),
    (1, 12, 1, 1, 8192, "none", None),
    (2, 8, 2, 3, 5000, "none", 7),
    (1, 12, 1, 4, 20000, "bottom_right", 0),
    (1, 32, 1, 2, 32768, "none", 0),
    (2, 12, 1, 16, 9000, "bottom_right", None),
]


@pytest.mark.parametrize("acc", ["fp32", "fp16"])
@pytest.mark.parametrize("b,hq,hkv,nq,nk,causal,splits", DECODE)
def test_packed_decode_vs_f64(library_path, b, hq, hkv, nq, nk, causal, splits, acc):
    say(f"case packed decode B{b} Hq{hq} Hkv{hkv} nq={nq} nk={nk} causal={causal} "
        f"splits={splits} acc={acc}")
    assert binding.query_tiles(b, hq, hkv, nq) == b * hkv
    q, k, v = draw(b, hq, hkv, nq, nk, seed=nq * 13 + nk)
    op = Operator(library_path, AttentionConfig(acc=acc, causal=causal, splits=splits))
    say(f"  parts per tile: {op.split_count(q.shape, k.shape)}")
    out, lse = op(q.cuda(), k.cuda(), v.cuda(), return_lse=True)
    torch.cuda.synchronize()
    out = out.float().cpu().numpy()
    check(out, orc.attention_f64(q, k, v, causal=causal), acc, "packed decode",
          orc.attention_f64(q, k, v.abs(), causal=causal))
    exact_lse = orc.lse_f64(q, k, causal=causal)
    check_lse(lse.cpu().numpy(), exact_lse, "packed decode")
    empty = np.isneginf(exact_lse)
    assert bool(np.all(out[empty] == 0)), "rows without keys must be exactly zero"


@pytest.mark.parametrize("acc", ["fp32", "fp16"])
def test_packed_debug_modes(library_path, acc):
    """Sync, trace and capture modes run the packed layout too: sync and
    trace return the production output bit for bit, trace writes one record
    per packed tile, and capture's final statistics give the output's lse."""
    b, hq, hkv, nq, nk = 2, 12, 1, 37, 1500
    say(f"case packed debug modes B{b} Hq{hq} Hkv{hkv} nq={nq} nk={nk} acc={acc}")
    q, k, v = (t.cuda() for t in draw(b, hq, hkv, nq, nk, seed=3))
    prod, lp = (t.clone() for t in Operator(library_path, AttentionConfig(acc=acc))(
        q, k, v, return_lse=True))
    sync, ls = Operator(library_path, AttentionConfig(acc=acc, sync=True))(q, k, v, return_lse=True)
    sync, ls = sync.clone(), ls.clone()
    traced = Operator(library_path, AttentionConfig(acc=acc, trace=True))
    tout = traced(q, k, v).clone()
    rec = traced.last["trace"].cpu().numpy()
    cap = Operator(library_path, AttentionConfig(acc=acc, capture=True))
    cout = cap(q, k, v).clone()
    stats = cap.last["stats"].cpu().numpy()
    torch.cuda.synchronize()
    assert torch.equal(prod, sync) and torch.equal(lp, ls)
    assert torch.equal(prod, tout)
    # 37 positions x 12 heads = 444 rows: 2 tiles per (batch, KV head), not 24.
    assert rec.shape == (binding.query_tiles(b, hq, hkv, nq), 8) and rec.shape[0] == b * hkv * 2
    assert np.array_equal(rec[:, 5], np.arange(rec.shape[0]))
    check(cout.float().cpu().numpy(), orc.attention_f64(q.cpu(), k.cpu(), v.cpu()), acc,
          "packed capture")
    # After the last block: lse = m + ln l per row, for every (b, h, row).
    m_last, l_last = stats[0, -1], stats[1, -1]
    lse_cap = (m_last + np.log(l_last)).reshape(b, hq, nq)
    err = np.abs(lse_cap - lp.cpu().numpy()).max()
    say(f"  capture lse vs output lse: {err:.3e}")
    assert err < 1e-4
