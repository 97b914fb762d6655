"""Trace mode and the MFMA ceiling kernel on the GPU.

Trace mode (fa_fwd_trace) is a separate instantiation of the production tile:
its O must equal the production kernel's bit for bit, and every query tile must
leave a well-formed record (its index, the key blocks it streamed, the block
size, monotonic clock stamps, a plausible clock and accelerator die). The
ceiling kernel must run, keep its sums finite, and report a plausible clock.
"""

import ctypes as C

import numpy as np
import pytest
import torch

from fa_amd import binding
from fa_amd.binding import AttentionConfig, Operator

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("acc", ["fp32", "fp16"])
@pytest.mark.parametrize("nq,nk,causal", [(1000, 900, "none"), (1024, 512, "bottom_right"),
                                          (600, 1100, "top_left")])
def test_trace_records_and_identical_output(library_path, acc, nq, nk, causal):
    from fa_amd.measure import clock

    say(f"case trace {acc} nq={nq} nk={nk} causal={causal}")
    g = torch.Generator().manual_seed(nq + nk)
    b, hq, hkv = 2, 6, 2
    q = torch.randn(b, hq, nq, 128, generator=g).half().cuda()
    k = torch.randn(b, hkv, nk, 128, generator=g).half().cuda()
    v = torch.randn(b, hkv, nk, 128, generator=g).half().cuda()
    plain = Operator(library_path, AttentionConfig(acc=acc, causal=causal))
    traced = Operator(library_path, AttentionConfig(acc=acc, causal=causal, trace=True))
    want = plain(q, k, v).clone()
    got = traced(q, k, v)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    rec = traced.last["trace"].cpu().numpy()
    # nq = 600 packs the 3 query heads of each KV head into 8 tiles per
    # (batch, KV head) instead of 3 x 3 per (batch, query head).
    tiles = binding.query_tiles(b, hq, hkv, nq)
    assert rec.shape == (tiles, 8)
    assert tiles < b * hq * -(-nq // 256) or nq != 600
    assert np.array_equal(rec[:, 5], np.arange(rec.shape[0]))
    bn = int(rec[0, 7])
    assert bn in (64, 128) and np.all(rec[:, 7] == bn)
    nblk_all = -(-nk // bn)
    if causal == "none":
        assert np.all(rec[:, 6] == nblk_all)
    else:
        assert np.all((rec[:, 6] >= 0) & (rec[:, 6] <= nblk_all))
        if causal == "bottom_right":
            assert np.any(rec[:, 6] == 0)          # tiles whose rows see no key
    assert np.all(rec[:, 2] >= rec[:, 1]) and np.all(rec[:, 4] >= rec[:, 3])
    assert np.all(((rec[:, 0] >> 32) & 15) < 8)   # one of the 8 accelerator dies
    mhz = clock.clocks_mhz(rec[rec[:, 6] > 0])
    assert mhz.size and np.all((mhz > 100) & (mhz < 3000)), mhz


def test_ceiling_kernel_runs_and_reports_a_clock():
    from fa_amd.measure import ceiling, clock

    say("case MFMA ceiling kernel, every mode, 256 workgroups")
    lib = ceiling._library()
    # Host-side rejections (nothing is launched): unknown mode, no
    # workgroups, misaligned operands.
    assert lib.fa_ceiling_mfma(13, 1, 1, C.c_void_p(16), C.c_void_p(16), None, None) == 1
    assert lib.fa_ceiling_threads(13) == 0 and lib.fa_ceiling_threads(6) == 256
    assert lib.fa_ceiling_threads(0) == 512
    assert lib.fa_ceiling_flops(0, 3) == lib.fa_ceiling_flops_per_workgroup(3)
    assert lib.fa_ceiling_flops(5, 3) * 2 == lib.fa_ceiling_flops_per_workgroup(3)
    assert lib.fa_ceiling_mfma(-1, 1, 1, C.c_void_p(16), C.c_void_p(16), None, None) == 1
    assert lib.fa_ceiling_mfma(0, 0, 1, C.c_void_p(16), C.c_void_p(16), None, None) == 1
    assert lib.fa_ceiling_mfma(0, 1, 1, C.c_void_p(24), C.c_void_p(16), None, None) == 1
    for mode, _ in ceiling.MODES:
        rate, records = ceiling.mfma_loop(mode, workgroups=256, iters=256, reps=1, warmup=1)
        s = clock.summarize(records)
        say(f"  mode {mode}: {rate:.1f} TFLOP/s at {s['median_mhz']:.0f} MHz")
        assert 10 < rate < 2600
        assert 100 < s["median_mhz"] < 3000
        assert np.all(records[:, 6] == 256)
        assert np.all(records[:, 7] == (64 if mode >= 7 else 16))
