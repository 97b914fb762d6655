"""fa_fwd_noalloc: the entry point that allocates nothing.

Its workspace is the library's static device array (FA_NOALLOC_SCRATCH_BYTES
per GPU). Called through the C ABI, it must give exactly fa_fwd's output (the
same kernels, only the workspace differs), on two calls in a row, the second
with a smaller input (ragged ones, which also use the padded copies in the
scratch, through both V layouts), and refuse problems whose workspace exceeds the array before any
work is enqueued. Captured in a HIP graph after a first eager call, its
replays must equal fa_fwd on the same inputs.
"""

import ctypes as C

import pytest
import torch

from fa_amd import binding

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


def inputs(b, hq, hkv, nq, nk, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, nq, 128, generator=g).half().cuda()
    k = torch.randn(b, hkv, nk, 128, generator=g).half().cuda()
    v = torch.randn(b, hkv, nk, 128, generator=g).half().cuda()
    return q, k, v


def with_workspace(lib, prob, q, k, v):
    """fa_fwd with a workspace torch allocated (the existing entry point)."""
    size = C.c_uint64()
    assert lib.fa_fwd_workspace_bytes(C.byref(prob), C.byref(size)) == 0
    ws = torch.empty(max(size.value, 16), dtype=torch.uint8, device="cuda")
    out = torch.empty_like(q)
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.fa_fwd(C.byref(prob), q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                      ws.data_ptr(), ws.numel(), C.c_void_p(stream)) == 0
    torch.cuda.synchronize()
    return out


def without_workspace(lib, prob, q, k, v):
    out = torch.empty_like(q)
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.fa_fwd_noalloc(C.byref(prob), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                            out.data_ptr(), C.c_void_p(stream))
    assert rc == 0, lib.fa_strerror(rc)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("acc", [0, 1])
def test_noalloc_matches_fa_fwd_on_two_calls(library_path, acc):
    lib = binding.load_library(library_path)
    # Second call smaller and ragged (V^T and a padded K in the scratch);
    # third smaller still, few query rows per KV head (the natural-V tile:
    # padded K and V copies in the scratch).
    shapes = [(2, 12, 1, 4096, 4096), (1, 6, 2, 700, 1000), (1, 8, 2, 100, 999)]
    for i, (b, hq, hkv, nq, nk) in enumerate(shapes):
        say(f"case noalloc acc={acc} call {i}: B={b} Hq={hq} Hkv={hkv} Nq={nq} Nk={nk}")
        q, k, v = inputs(b, hq, hkv, nq, nk, seed=10 * i + acc)
        prob = binding.FaProblem(b, hq, hkv, nq, nk, 128, 128 ** -0.5, acc, 0, 0)
        got = without_workspace(lib, prob, q, k, v)
        want = with_workspace(lib, prob, q, k, v)
        assert torch.equal(got, want), (acc, i)
        assert torch.isfinite(got.float()).all()


def test_noalloc_headline_size_fits_and_oversize_is_refused(library_path):
    lib = binding.load_library(library_path)
    size = C.c_uint64()
    c3 = binding.FaProblem(2, 12, 1, 131072, 131072, 128, 128 ** -0.5, 0, 0, 0)
    assert lib.fa_fwd_workspace_bytes(C.byref(c3), C.byref(size)) == 0
    assert size.value <= binding.NOALLOC_SCRATCH_BYTES
    big = binding.FaProblem(4, 12, 1, 256, 131071, 128, 128 ** -0.5, 0, 0, 0)   # ragged: 256 MiB
    # No tensors: the size check comes before the null check, so the refusal
    # is FA_ERR_SCRATCH, and a regression would return FA_ERR_NULL without
    # enqueuing anything.
    assert lib.fa_fwd_noalloc(C.byref(big), None, None, None, None, None) == 14
    assert b"scratch" in lib.fa_strerror(14)


def test_noalloc_captured_in_a_graph_replays_like_eager_calls(library_path):
    """fa_fwd_noalloc captured in a HIP graph (after a first eager call on the
    device, as the header asks): every replay, with eager work and new input
    values between replays, equals fa_fwd on the same inputs bit for bit."""
    lib = binding.load_library(library_path)
    b, hq, hkv, nq, nk = 1, 12, 1, 1024, 1000          # ragged keys: prep + attention kernels
    say(f"case noalloc graph: B={b} Hq={hq} Hkv={hkv} Nq={nq} Nk={nk}")
    prob = binding.FaProblem(b, hq, hkv, nq, nk, 128, 128 ** -0.5, 0, 0, 0)
    sets = [inputs(b, hq, hkv, nq, nk, seed=s) for s in (21, 22)]
    want = [with_workspace(lib, prob, *x) for x in sets]
    q, k, v = (t.clone() for t in sets[0])
    out = torch.empty_like(q)
    without_workspace(lib, prob, q, k, v)                # first call: host-side set-up
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = lib.fa_fwd_noalloc(C.byref(prob), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                out.data_ptr(), C.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, lib.fa_strerror(rc)
    for replay in range(4):
        src = sets[replay % 2]
        for dst, t in zip((q, k, v), src):
            dst.copy_(t)
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        say(f"  replay {replay}")
        assert torch.equal(out, want[replay % 2]), replay
    del graph
