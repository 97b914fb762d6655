"""The C-ABI library loads, exports every declared symbol, and validates on the host.

No compute call runs here: every call below returns an error code before the
library touches the HIP runtime, so the suite runs without a GPU.
"""

import ctypes as C
import re
from pathlib import Path

import pytest

from fa_amd import binding

HEADER = Path(__file__).resolve().parent.parent / "include" / "fa_hip.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(fa_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_binding_signatures():
    assert declared_functions() == sorted(binding.SIGNATURES)


def test_library_exports_every_declared_symbol(library_path):
    lib = C.CDLL(library_path, mode=C.RTLD_LOCAL)
    for name in declared_functions():
        assert hasattr(lib, name), name
    binding.load_library(library_path)


def problem(**kw):
    base = dict(batch=1, heads_q=12, heads_kv=1, seq_q=4096, seq_k=4096, dim=128,
                scale=128 ** -0.5, acc=0, kernel=0, causal=0)
    base.update(kw)
    return binding.FaProblem(**base)


def ws_bytes(lib, prob):
    size = C.c_uint64(0)
    rc = lib.fa_fwd_workspace_bytes(C.byref(prob), C.byref(size))
    return rc, size.value


@pytest.fixture(scope="module")
def lib(library_path):
    return binding.load_library(library_path)


def test_workspace_size(lib):
    # Many query rows per KV head (12 x 4096): the V^T tile, whose workspace
    # holds V^T, plus 256 bytes for the work-queue counter.
    rc, size = ws_bytes(lib, problem(batch=2, heads_kv=1, seq_k=131072))
    assert rc == 0 and size == 2 * 1 * 131072 * 128 * 2 + 256
    # A ragged key tail adds the zero-padded K.
    rc, size = ws_bytes(lib, problem(seq_k=1000))
    assert rc == 0 and size == 2 * 1024 * 128 * 2 + 256
    # Few query rows per KV head (2 x 512): the natural-V tile reads K and V
    # where they lie, so only the counter.
    rc, size = ws_bytes(lib, problem(heads_q=8, heads_kv=4, seq_q=512, seq_k=1024))
    assert rc == 0 and size == 256
    # A ragged key tail adds zero-padded copies of K and V for every KV head.
    rc, size = ws_bytes(lib, problem(heads_q=8, heads_kv=4, seq_q=512, seq_k=1000))
    assert rc == 0 and size == 2 * 4 * 1024 * 128 * 2 + 256
    # Forcing either tile gives its own layout whatever the shape.
    assert ws_bytes(lib, problem(batch=2, seq_k=131072, kernel=4)) == (0, 256)
    assert ws_bytes(lib, problem(heads_q=8, heads_kv=4, seq_q=512, seq_k=1024, kernel=3)) == \
        (0, 4 * 1024 * 128 * 2 + 256)


@pytest.mark.parametrize("kw,code", [
    (dict(batch=0), 2), (dict(heads_q=12, heads_kv=5), 2), (dict(seq_k=-64), 2),
    (dict(dim=64), 3), (dict(acc=2), 7), (dict(scale=0.0), 8), (dict(scale=float("inf")), 8),
    (dict(kernel=99), 9), (dict(kernel=-1), 9), (dict(causal=3), 12), (dict(causal=-1), 12),
    (dict(seq_q=1 << 30), 2),
])
def test_geometry_errors(lib, kw, code):
    rc, _ = ws_bytes(lib, problem(**kw))
    assert rc == code
    assert lib.fa_strerror(rc)


def test_ragged_tails_and_workspace(lib):
    # The automatic choice masks ragged tails, so any Nq, Nk >= 1 is valid;
    # a ragged key tail adds zero-padded copies (whole blocks of the 128-key
    # tile): of K and V for the natural-V tile (few query rows per KV head),
    # of K beside V^T for the V^T tile (many), two copies either way.
    for nq, nk in ((1, 1), (300, 1000), (4097, 4095), (256, 129)):
        rc, size = ws_bytes(lib, problem(seq_q=nq, seq_k=nk))
        assert rc == 0, (nq, nk)
        pad = -(-nk // 128) * 128
        assert size == 2 * pad * 128 * 2 + 256, (nq, nk, size)
    rc, size = ws_bytes(lib, problem(seq_q=100, seq_k=4096))
    assert rc == 0 and size == 256                     # natural V, no key tail: the counter
    rc, size = ws_bytes(lib, problem(seq_q=4096, seq_k=4096))
    assert rc == 0 and size == 4096 * 128 * 2 + 256    # V^T, no key tail: V^T and the counter
    # A 64-key tile pads to whole 64-key blocks.
    rc, size = ws_bytes(lib, problem(seq_q=300, seq_k=1000, kernel=1))
    assert rc == 0 and size == 2 * 1024 * 128 * 2 + 256
    for kernel in range(lib.fa_kernel_count() + 1):      # every tile masks tails
        rows, keys = C.c_int32(), C.c_int32()
        assert lib.fa_fwd_tile(C.byref(problem(kernel=kernel)), C.byref(rows), C.byref(keys)) == 0
        assert (rows.value, keys.value) == (1, 1)


def test_causal_selection(lib):
    # Every tile applies causal masks, whatever the shape.
    for causal in (1, 2):
        for nq, nk in ((4096, 4096), (300, 1000), (1000, 7)):
            for acc in (0, 1):
                prob = problem(seq_q=nq, seq_k=nk, causal=causal, acc=acc)
                idx = C.c_int32()
                assert lib.fa_fwd_select(C.byref(prob), C.byref(idx)) == 0
                assert lib.fa_kernel_name(idx.value).startswith(b"pp_"), (causal, nq, nk, acc)
                assert ws_bytes(lib, prob)[0] == 0
        for kernel in range(1, lib.fa_kernel_count() + 1):
            assert ws_bytes(lib, problem(causal=causal, kernel=kernel))[0] == 0
    assert b"causal" in lib.fa_strerror(12)
    with pytest.raises(ValueError):
        binding.AttentionConfig(causal="diagonal")
    assert binding.make_problem((1, 2, 8, 128), (1, 1, 8, 128), 1.0,
                                binding.AttentionConfig(causal="bottom_right")).causal == 2


def test_key_length_limit(lib):
    # A head's K and V rows are addressed with 32-bit byte offsets: Nk' keys x 256 B < 2^31.
    assert ws_bytes(lib, problem(seq_q=256, seq_k=8_000_000))[0] == 0
    assert ws_bytes(lib, problem(seq_q=256, seq_k=9_000_000))[0] == 2


def test_capture_count_and_rejections(lib):
    prob = problem(seq_q=300, seq_k=1000)            # FP32 default tile: 128-key blocks
    count, block = C.c_uint64(), C.c_int32()
    assert lib.fa_fwd_capture_count(C.byref(prob), C.byref(count), C.byref(block)) == 0
    assert block.value == 128 and count.value == 4 * 8 * 12 * 300
    prob64 = problem(seq_q=300, seq_k=1000, acc=1, kernel=1)   # a 64-key tile
    assert lib.fa_fwd_capture_count(C.byref(prob64), C.byref(count), C.byref(block)) == 0
    assert block.value == 64 and count.value == 4 * 16 * 12 * 300
    assert lib.fa_fwd_capture_count(C.byref(prob), None, C.byref(block)) == 1
    # Launch-time checks happen on the host, before any GPU work.
    p = C.c_void_p(4096)
    _, size = ws_bytes(lib, prob)
    need = 4 * 8 * 12 * 300
    assert lib.fa_fwd_capture(C.byref(prob), p, p, p, p, None, None, need, p, size, None) == 1
    assert lib.fa_fwd_capture(C.byref(prob), p, p, p, p, None, p, need - 1, p, size, None) == 11
    assert lib.fa_strerror(11)


def test_trace_count_and_rejections(lib):
    # One 8-word record per query tile. Nq = 300 rows of 12 query heads that
    # share one KV head pack into ceil(3600 / 256) = 15 tiles per batch
    # instead of 12 x 2 (position-major rows of the whole group).
    prob = problem(batch=2, seq_q=300, seq_k=1000)
    count = C.c_uint64()
    assert lib.fa_fwd_trace_count(C.byref(prob), C.byref(count)) == 0
    assert count.value == 8 * 2 * 15
    assert lib.fa_fwd_trace_count(C.byref(prob), None) == 1
    assert lib.fa_fwd_trace_count(C.byref(problem(dim=64)), C.byref(count)) == 3
    p = C.c_void_p(4096)
    _, size = ws_bytes(lib, prob)
    need = 8 * 2 * 15
    assert lib.fa_fwd_trace(C.byref(prob), p, p, p, p, None, need, p, size, None) == 1
    assert lib.fa_fwd_trace(C.byref(prob), p, p, p, p, p, need - 1, p, size, None) == 13
    assert lib.fa_fwd_trace(C.byref(prob), p, p, p, p, C.c_void_p(4104), need, p, size, None) == 5
    assert b"trace" in lib.fa_strerror(13)
    with pytest.raises(ValueError):
        binding.AttentionConfig(trace=True, capture=True)


@pytest.mark.parametrize("b,hq,hkv,nq", [
    (1, 12, 1, 1), (1, 12, 1, 21), (1, 12, 1, 22), (2, 12, 1, 255), (1, 12, 1, 256),
    (1, 12, 1, 4096), (2, 12, 1, 300), (2, 6, 2, 600), (2, 6, 2, 1000), (1, 8, 2, 40),
    (3, 4, 4, 7), (1, 1, 1, 1), (1, 64, 8, 3), (1, 32, 1, 100), (2, 2, 1, 129)])
def test_query_tiles_match_the_library(lib, b, hq, hkv, nq):
    # The binding's tile rule is the library's: packed only when it needs
    # fewer tiles (never for a group of 1 or 256-row multiples per head).
    count = C.c_uint64()
    assert lib.fa_fwd_trace_count(C.byref(problem(batch=b, heads_q=hq, heads_kv=hkv, seq_q=nq,
                                                  seq_k=512)), C.byref(count)) == 0
    assert count.value == 8 * binding.query_tiles(b, hq, hkv, nq)
    plain = b * hq * -(-nq // 256)
    assert binding.query_tiles(b, hq, hkv, nq) <= plain
    if hq == hkv or nq % 256 == 0:
        assert binding.query_tiles(b, hq, hkv, nq) == plain


def test_packed_decode_split_choice(lib):
    # One query row per head, 12 heads on one KV head: one packed tile, so
    # the automatic split spreads its 1024 key blocks over many CUs.
    rc, n = split_count(lib, problem(seq_q=1, seq_k=131072), 0)
    assert rc == 0 and n >= 32, n


def test_sync_mode_rejections(lib):
    # fa_fwd_sync validates like fa_fwd_lse before anything is launched.
    prob = problem(batch=2, seq_q=300, seq_k=1000)
    p = C.c_void_p(4096)
    _, size = ws_bytes(lib, prob)
    assert lib.fa_fwd_sync(C.byref(prob), None, p, p, p, None, p, size, None) == 1
    assert lib.fa_fwd_sync(C.byref(prob), p, p, p, p, None, p, size - 1, None) == 6
    assert lib.fa_fwd_sync(C.byref(prob), p, p, p, p, C.c_void_p(4100), p, size, None) == 5
    assert lib.fa_fwd_sync(C.byref(problem(dim=64)), p, p, p, p, None, p, size, None) == 3
    assert binding.AttentionConfig(sync=True).sync
    for bad in ({"sync": True, "trace": True}, {"sync": True, "capture": True}, {"sync": 1}):
        with pytest.raises(ValueError):
            binding.AttentionConfig(**bad)


def test_fwd_rejects_before_launch(lib):
    prob = problem()
    # NULL tensors, missing workspace and misaligned pointers fail on the host.
    assert lib.fa_fwd(C.byref(prob), None, None, None, None, None, 0, None) == 1
    p = C.c_void_p(4096)
    assert lib.fa_fwd(C.byref(prob), p, p, p, p, None, 0, None) == 6
    _, size = ws_bytes(lib, prob)
    assert lib.fa_fwd(C.byref(prob), p, p, p, p, p, size - 1, None) == 6
    odd = C.c_void_p(4096 + 8)
    assert lib.fa_fwd(C.byref(prob), p, odd, p, p, p, size, None) == 5
    assert lib.fa_fwd(None, p, p, p, p, p, size, None) == 1
    # fa_fwd_lse: same checks, plus the lse pointer's alignment (NULL is allowed).
    assert lib.fa_fwd_lse(C.byref(prob), p, p, p, p, odd, p, size, None) == 5
    assert lib.fa_fwd_lse(C.byref(prob), None, p, p, p, None, p, size, None) == 1
    # A stream must belong to the current device (checked at launch, after the
    # host-side checks above); the code has its own message.
    assert b"device" in lib.fa_strerror(16)


def test_kernel_table(lib):
    n = lib.fa_kernel_count()
    assert n == 4
    names = [lib.fa_kernel_name(i).decode() for i in range(1, n + 1)]
    assert len(set(names)) == n
    assert lib.fa_kernel_name(0) is None and lib.fa_kernel_name(n + 1) is None
    for i in range(0, n + 1):
        rows, keys = C.c_int32(), C.c_int32()
        assert lib.fa_fwd_tile(C.byref(problem(kernel=i)), C.byref(rows), C.byref(keys)) == 0
        assert (rows.value, keys.value) == (1, 1)
        sel = C.c_int32()
        assert lib.fa_fwd_select(C.byref(problem(kernel=i)), C.byref(sel)) == 0
        assert (sel.value == i) if i else (1 <= sel.value <= n)
    sel = C.c_int32()
    assert lib.fa_fwd_select(C.byref(problem(kernel=n + 1)), C.byref(sel)) == 9
    assert lib.fa_fwd_select(None, C.byref(sel)) == 1


def test_automatic_choice_on_invalid_geometry(lib):
    # The automatic choice looks at query rows per KV head; for a geometry
    # validation rejects (no KV head, a group that does not divide) it must
    # not divide by zero: fa_fwd_select still names a tile, and the calls
    # that validate report the geometry error.
    sel = C.c_int32()
    for kw in (dict(heads_kv=0), dict(heads_q=12, heads_kv=5), dict(seq_q=0), dict(heads_q=0)):
        assert lib.fa_fwd_select(C.byref(problem(**kw)), C.byref(sel)) == 0, kw
        assert lib.fa_kernel_name(sel.value) == b"pp_n128_r2", kw
        assert ws_bytes(lib, problem(**kw))[0] == 2, kw


def test_automatic_choice(lib):
    # kernel = 0: the 128-key tile for both accumulators, reading V^T with
    # more than 2048 query rows per KV head (group x Nq) and V in its
    # natural layout with at most that many.
    sel = C.c_int32()
    cases = [(12, 1, 4096, b"pp_n128_r2"), (12, 1, 131072, b"pp_n128_r2"), (12, 1, 1000, b"pp_n128_r2"),
             (12, 1, 171, b"pp_n128_r2"), (12, 1, 170, b"pp_n128_r2_vnat"), (12, 1, 1, b"pp_n128_r2_vnat"),
             (8, 8, 2048, b"pp_n128_r2_vnat"), (8, 8, 2049, b"pp_n128_r2"), (64, 8, 16, b"pp_n128_r2_vnat")]
    for hq, hkv, seq, name in cases:
        for acc in (0, 1):
            prob = problem(heads_q=hq, heads_kv=hkv, seq_q=seq, seq_k=seq, acc=acc)
            assert lib.fa_fwd_select(C.byref(prob), C.byref(sel)) == 0
            assert lib.fa_kernel_name(sel.value) == name, (hq, hkv, seq)


def test_operator_validation_without_gpu(library_path):
    import torch

    op = binding.Operator(library_path)
    q = torch.zeros(1, 12, 256, 128, dtype=torch.float16)
    k = torch.zeros(1, 1, 256, 128, dtype=torch.float16)
    with pytest.raises(ValueError, match="GPU"):
        op(q, k, k)
    with pytest.raises(ValueError, match="geometry"):
        op(q, torch.zeros(1, 5, 256, 128, dtype=torch.float16),
           torch.zeros(1, 5, 256, 128, dtype=torch.float16))
    with pytest.raises(ValueError, match=r"\[B,H,N,128\]"):
        op(q[0], k, k)
    with pytest.raises(ValueError):
        binding.AttentionConfig(acc="bf16")


def test_strided_validation(lib):
    # Layout errors are reported before anything is launched.
    prob = problem(heads_q=4, seq_q=256, seq_k=256)
    fake = C.c_void_p(256)

    def call(**over):
        st = binding.FaStrides()
        vals = dict(q=(4 * 256 * 128, 256 * 128, 128), k=(256 * 128, 256 * 128, 128),
                    v=(256 * 128, 256 * 128, 128), o=(4 * 256 * 128, 256 * 128, 128))
        vals.update(over)
        for name, t in vals.items():
            getattr(st, name)[:] = t
        return lib.fa_fwd_strided(C.byref(prob), C.byref(st), fake, fake, fake, fake, None, fake,
                                  1 << 30, None)

    assert lib.fa_fwd_strided(C.byref(prob), None, fake, fake, fake, fake, None, fake, 1 << 30,
                              None) == 1
    assert call(q=(4 * 256 * 128, 256 * 128, 132)) == 5          # row stride not a multiple of 8
    assert call(k=(256 * 128, -8, 128)) == 2                     # negative stride
    assert call(o=(4 * 256 * 128, 256 * 128, 64)) == 2           # rows overlap
    assert call(k=(0, 0, 1 << 23), v=(0, 0, 128)) == 2           # key rows span >= 2^31 bytes
    assert call(v=(0, 0, 1 << 23)) == 2                          # so do the value rows


def test_noalloc_rejects_before_touching_the_gpu(lib):
    # Problems whose workspace exceeds the static scratch (64 MiB) and NULL
    # tensors are refused on the host: here V^T and a padded K, 2 * 4 *
    # 131072 keys * 256 B = 256 MiB.
    fake = C.c_void_p(4096)
    big = problem(batch=4, seq_q=256, seq_k=131071)
    assert lib.fa_fwd_noalloc(C.byref(big), fake, fake, fake, fake, None) == 14
    rc, size = ws_bytes(lib, problem(batch=4, seq_q=16, seq_k=131072))   # natural V: the counter
    assert rc == 0 and size == 256
    assert lib.fa_fwd_noalloc(C.byref(problem(dim=64)), fake, fake, fake, fake, None) == 3
    assert lib.fa_fwd_noalloc(C.byref(problem()), None, fake, fake, fake, None) == 1
    assert lib.fa_fwd_noalloc(None, fake, fake, fake, fake, None) == 1
    # The headline configuration (B=2, Nk=131072, no key tail) fits.
    rc, size = ws_bytes(lib, problem(batch=2, seq_q=131072, seq_k=131072))
    assert rc == 0 and size <= binding.NOALLOC_SCRATCH_BYTES


def split_count(lib, prob, splits, cus=256):
    n = C.c_int32(-1)
    rc = lib.fa_fwd_split_count(C.byref(prob), splits, cus, C.byref(n))
    return rc, n.value


def split_ws(lib, prob, splits):
    size = C.c_uint64(0)
    rc = lib.fa_fwd_split_workspace_bytes(C.byref(prob), splits, C.byref(size))
    return rc, size.value


def test_split_count_choice(lib):
    # Automatic choice on a 256-CU GPU: grids with at least 2 x 256 tiles are
    # never split; 12 query tiles against 131072 keys are; c0 (192 tiles of
    # 32 key blocks, one round) gains too little from splitting to pay for
    # the merge.
    assert split_count(lib, problem(batch=2, seq_q=131072, seq_k=131072), 0) == (0, 1)
    assert split_count(lib, problem(seq_q=4096, seq_k=4096), 0) == (0, 1)
    rc, n = split_count(lib, problem(seq_q=256, seq_k=131072), 0)
    assert rc == 0 and 16 <= n <= 64, n
    # Causal masks: the choice looks at the key blocks each tile sees. One
    # bottom-right query tile at the end of 131072 keys sees them all and is
    # split; the causal headline shape has tiles enough.
    rc, n = split_count(lib, problem(seq_q=256, seq_k=131072, causal=2), 0)
    assert rc == 0 and n > 1
    assert split_count(lib, problem(batch=2, seq_q=131072, seq_k=131072, causal=1), 0) == (0, 1)
    # Top-left, Nq = Nk = 1024 on 4 CUs: 4 tiles of 2, 4, 6 and 8 blocks. The
    # 8-block tile alone bounds the launch at 9.5 block times; two parts per
    # tile (blocks 0-3, 4-7) bring it to ~7.3 with the merge, so 2 is taken.
    assert split_count(lib, problem(heads_q=1, seq_q=1024, seq_k=1024, causal=1), 0, cus=4) == (0, 2)
    # Full attention: the modelled best count. 24 tiles of 512 key blocks on
    # 256 CUs: 10 parts are 240 items in one round of 51.2 + 1.5 block
    # times; 11 would need a second round.
    assert split_count(lib, problem(seq_q=512, seq_k=65536), 0) == (0, 10)
    # Explicit counts are clamped to the key blocks (128-key tile: 1000 keys
    # are 8 blocks) and do not depend on the CU count.
    assert split_count(lib, problem(seq_k=1000), 100) == (0, 8)
    assert split_count(lib, problem(seq_k=1000), 3, cus=1) == (0, 3)
    assert split_count(lib, problem(seq_k=1000), 1) == (0, 1)
    # Errors: counts outside 0..1024, a negative CU count, bad geometry.
    assert split_count(lib, problem(), -1)[0] == 15
    assert split_count(lib, problem(), 1025)[0] == 15
    assert split_count(lib, problem(), 2, cus=-1)[0] == 15
    assert split_count(lib, problem(dim=64), 2)[0] == 3
    assert lib.fa_fwd_split_count(C.byref(problem()), 2, 256, None) == 1


def test_split_workspace(lib):
    # One part: fa_fwd_workspace_bytes. n parts add the parts' lse (FP32
    # [n][R], padded to 256 bytes) and O (FP32 [n][R][128]), R = B * Hq * Nq.
    prob = problem(batch=1, heads_q=12, seq_q=300, seq_k=4096)
    _, base = ws_bytes(lib, prob)
    assert split_ws(lib, prob, 1) == (0, base)
    rows = 12 * 300
    for n in (2, 5, 32):
        lp = (n * rows * 4 + 255) // 256 * 256
        assert split_ws(lib, prob, n) == (0, base + lp + n * rows * 128 * 4)
    # Clamped like the count: 4096 keys are 32 blocks of 128.
    assert split_ws(lib, prob, 100) == split_ws(lib, prob, 32)
    assert split_ws(lib, prob, -3)[0] == 15
    assert lib.fa_fwd_split_workspace_bytes(C.byref(prob), 2, None) == 1


def test_split_rejects_before_launch(lib):
    prob = problem(seq_q=256, seq_k=8192)
    p = C.c_void_p(4096)
    _, size = split_ws(lib, prob, 4)
    assert lib.fa_fwd_split(C.byref(prob), 4, None, None, p, p, p, None, p, size, None) == 1
    assert lib.fa_fwd_split(C.byref(prob), 4, None, p, p, p, p, None, p, size - 1, None) == 6
    assert lib.fa_fwd_split(C.byref(prob), 4, None, p, p, p, p, C.c_void_p(4100), p, size,
                            None) == 5
    assert lib.fa_fwd_split(C.byref(prob), -1, None, p, p, p, p, None, p, size, None) == 15
    assert lib.fa_fwd_split(C.byref(problem(dim=64)), 4, None, p, p, p, p, None, p, size,
                            None) == 3
    bad = binding.FaStrides()
    for name in ("q", "k", "v", "o"):
        getattr(bad, name)[:] = (256 * 128, 256 * 128, 132)
    assert lib.fa_fwd_split(C.byref(prob), 4, C.byref(bad), p, p, p, p, None, p, size,
                            None) == 5
    # The binding's configuration checks.
    assert binding.AttentionConfig(splits=0).splits == 0
    for bad_cfg in ({"splits": -1}, {"splits": 1025}, {"splits": 2.0}, {"splits": True},
                    {"splits": 2, "sync": True}, {"splits": 2, "capture": True},
                    {"splits": 0, "trace": True}):
        with pytest.raises(ValueError):
            binding.AttentionConfig(**bad_cfg)


def test_host_sanitizer_build_leaves_device_code_alone():
    """The opt-in host-sanitizer target (python -m fa_amd.build --sanitize)
    puts every -fsanitize= behind -Xarch_host, so no GPU code is built with
    a sanitizer, and the default builds never include it."""
    from fa_amd import build

    flags = build.HOSTSAN.flags
    sanitizers = [i for i, f in enumerate(flags) if f.startswith("-fsanitize")]
    assert sanitizers and all(flags[i - 1] == "-Xarch_host" for i in sanitizers)
    assert not any(f.startswith("-fsanitize") for f in build.FLAGS)
    assert build.HOSTSAN not in build.TARGETS
    assert build.HOSTSAN.library != build.LIBRARY
    assert build.identity(build.HOSTSAN) != build.identity(build.ATTENTION)
