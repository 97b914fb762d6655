"""The two V layouts of the 128-key tile give identical results.

pp_n128_r2 reads V^T, the key-permuted transposed copy the prep kernel
writes; pp_n128_r2_vnat reads V where it lies, staged in LDS as [key][dim]
rows and turned into the same matrix operand by transposing LDS reads
(ds_read_b64_tr_b16). Both feed the matrix cores the same values in the same
order, so every output and lse must be equal bit for bit. The V^T tile is
checked against the float64 oracle throughout the suite, which pins the
natural-V tile too. Covered here: full and causal masks, ragged query and key
tails, packed grouped-query tiles, the key-split forward, both accumulators,
K and V with different strides (the natural-V tile reads V through its own),
and the sync, capture and trace modes. Every case prints its name before its
GPU work.
"""

import numpy as np
import pytest
import torch

from fa_amd import binding
from fa_amd.binding import AttentionConfig, Operator
from oracle import attention as orc

from test_gpu_parity import check, say

pytestmark = pytest.mark.gpu

VT, VNAT = 3, 4      # tile configurations pp_n128_r2 and pp_n128_r2_vnat


def test_tile_numbers(library_path):
    lib = binding.load_library(library_path)
    assert lib.fa_kernel_name(VT) == b"pp_n128_r2" and lib.fa_kernel_name(VNAT) == b"pp_n128_r2_vnat"


def draw(b, hq, hkv, nq, nk, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(b, hq, nq, 128, generator=g).half().cuda(),
            torch.randn(b, hkv, nk, 128, generator=g).half().cuda(),
            torch.randn(b, hkv, nk, 128, generator=g).half().cuda())


def both(lib, q, k, v, **cfg):
    """(out, lse) of the V^T tile and of the natural-V tile."""
    res = []
    for kernel in (VT, VNAT):
        out, lse = Operator(lib, AttentionConfig(kernel=kernel, **cfg))(q, k, v, return_lse=True)
        res.append((out.clone(), lse.clone()))
    torch.cuda.synchronize()
    return res


# (B, Hq, Hkv, Nq, Nk, causal, splits): full and causal masks, ragged tails,
# packed decode tiles, the key-split forward (None: one pass, 0: automatic).
CASES = [
    (2, 12, 1, 1024, 2048, "none", None),
    (1, 12, 1, 300, 1000, "top_left", None),
    (2, 8, 2, 3, 5000, "bottom_right", None),
    (1, 4, 4, 777, 129, "none", None),
    (1, 12, 1, 1, 65536, "none", 0),
    (2, 12, 1, 256, 8192, "bottom_right", 5),
    (1, 64, 8, 2, 3000, "none", 0),
    (1, 6, 3, 1000, 1000, "top_left", 3),
]


@pytest.mark.parametrize("acc", ["fp32", "fp16"])
@pytest.mark.parametrize("b,hq,hkv,nq,nk,causal,splits", CASES)
def test_v_layouts_bit_equal(library_path, b, hq, hkv, nq, nk, causal, splits, acc):
    say(f"case v layouts B{b} Hq{hq} Hkv{hkv} nq={nq} nk={nk} causal={causal} splits={splits} acc={acc}")
    q, k, v = draw(b, hq, hkv, nq, nk, seed=nq * 11 + nk)
    (o3, l3), (o4, l4) = both(library_path, q, k, v, acc=acc, causal=causal, splits=splits)
    assert torch.isfinite(o4).all()
    diff = (o3.float() - o4.float()).abs().max().item()
    assert torch.equal(o3, o4), f"max |diff| {diff:.3e}"
    assert torch.equal(l3, l4)


@pytest.mark.parametrize("acc", ["fp32", "fp16"])
def test_v_layouts_with_distinct_k_and_v_strides(library_path, acc):
    """K as a [B, N, H, 128] view, V with rows padded to 200 elements and its
    KV head broadcast over a second one (stride 0): bit-equal between the
    layouts and to contiguous copies, and within the oracle's bound."""
    b, hq, hkv, nq, nk = 1, 8, 2, 200, 1500
    say(f"case v layouts strided K/V B{b} Hq{hq} Hkv{hkv} nq={nq} nk={nk} acc={acc}")
    g = torch.Generator().manual_seed(5)
    q = torch.randn(b, hq, nq, 128, generator=g).half().cuda()
    k = torch.randn(b, nk, hkv, 128, generator=g).half().cuda().transpose(1, 2)
    vwide = torch.randn(b, 1, nk, 200, generator=g).half().cuda()
    v = vwide[..., :128].expand(b, hkv, nk, 128)
    assert not k.is_contiguous() and not v.is_contiguous() and v.stride(1) == 0
    (o3, l3), (o4, l4) = both(library_path, q, k, v, acc=acc)
    (oc, lc), _ = both(library_path, q, k.contiguous(), v.contiguous(), acc=acc)
    assert torch.equal(o3, o4) and torch.equal(l3, l4)
    assert torch.equal(o4, oc) and torch.equal(l4, lc)
    check(o4.float().cpu().numpy(), orc.attention_f64(q.cpu(), k.cpu(), v.cpu()), acc, "strided vnat")


@pytest.mark.parametrize("acc", ["fp32", "fp16"])
def test_natural_v_debug_modes(library_path, acc):
    """Sync and trace runs of the natural-V tile return its production output
    bit for bit, and its capture statistics equal the V^T tile's."""
    b, hq, hkv, nq, nk = 1, 12, 1, 37, 1500
    say(f"case natural-V debug modes B{b} Hq{hq} Hkv{hkv} nq={nq} nk={nk} acc={acc}")
    q, k, v = draw(b, hq, hkv, nq, nk, seed=9)
    lib = library_path
    prod = Operator(lib, AttentionConfig(acc=acc, kernel=VNAT))(q, k, v).clone()
    sync = Operator(lib, AttentionConfig(acc=acc, kernel=VNAT, sync=True))(q, k, v).clone()
    traced = Operator(lib, AttentionConfig(acc=acc, kernel=VNAT, trace=True))
    tout = traced(q, k, v).clone()
    stats = []
    for kernel in (VT, VNAT):
        cap = Operator(lib, AttentionConfig(acc=acc, kernel=kernel, capture=True))
        cap(q, k, v)
        stats.append(cap.last["stats"].clone())
    torch.cuda.synchronize()
    assert torch.equal(prod, sync) and torch.equal(prod, tout)
    assert traced.last["trace"].shape[0] == binding.query_tiles(b, hq, hkv, nq)
    assert torch.equal(stats[0], stats[1])
    assert np.isfinite(stats[1].cpu().numpy()[1]).all()
