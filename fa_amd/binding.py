"""ctypes binding of ``libfa_hip.so``: public inputs q/k/v, public output O.

Mirrors the reference's operator binding
(``backends/cce_fa_nk_nz_vector_fp32_v5_sumpack/binding.py:6-110``):

  * the library is opened with ``RTLD_LOCAL``;
  * a call is two-phase: ``fa_fwd_workspace_bytes`` sizes the workspace,
    ``fa_fwd`` (or ``fa_fwd_lse`` when the per-row log-sum-exp is asked for)
    enqueues the forward on the current torch stream;
  * geometry, dtype, device and layout errors raise ``ValueError`` before any
    launch (any [B,H,N,128] view whose last dimension is contiguous and whose
    rows are 16-byte aligned is accepted: non-contiguous views, such as the
    sequence-major tensors of FlashAttention-style code, go through
    ``fa_fwd_strided`` without a copy); a nonzero library status raises ``RuntimeError("fa_fwd <where>:
    <status> (<message>)")``;
  * output and workspace tensors are allocated by torch, cached per
    (shapes, device, config), and the same cached output tensor is returned
    on every call; the workspace grows on demand. Calls of one ``Operator``
    therefore share its output and workspace: forwards that may overlap on
    different streams need an ``Operator`` each.

Nothing here falls back to another implementation: without the built library
construction fails.
"""

import ctypes as C
import math
from dataclasses import dataclass

FA_ACC = {"fp32": 0, "fp16": 1}
# Attention masks (enum fa_causal): full attention, the reference's only mode,
# or a causal mask aligned top-left (key j <= query i, torch's
# scaled_dot_product_attention(is_causal=True)) or bottom-right
# (j <= i + Nk - Nq).
FA_CAUSAL = {"none": 0, "top_left": 1, "bottom_right": 2}
# 64-bit words per query-tile record of trace mode (fa_fwd_trace).
TRACE_WORDS = 8
# Workspace bytes fa_fwd_noalloc's static device array holds (FA_NOALLOC_SCRATCH_BYTES).
NOALLOC_SCRATCH_BYTES = (64 << 20) + (64 << 10)


class FaProblem(C.Structure):
    _fields_ = [
        ("batch", C.c_int64),
        ("heads_q", C.c_int64),
        ("heads_kv", C.c_int64),
        ("seq_q", C.c_int64),
        ("seq_k", C.c_int64),
        ("dim", C.c_int64),
        ("scale", C.c_float),
        ("acc", C.c_int32),
        ("kernel", C.c_int32),
        ("causal", C.c_int32),
    ]


class FaStrides(C.Structure):
    """Element strides of dims B, H, N of q, k, v and o (``fa_strides``)."""
    _fields_ = [("q", C.c_int64 * 3), ("k", C.c_int64 * 3), ("v", C.c_int64 * 3),
                ("o", C.c_int64 * 3)]


# Every symbol include/fa_hip.h declares, with its ctypes signature.
SIGNATURES = {
    "fa_fwd_workspace_bytes": (C.c_int, [C.POINTER(FaProblem), C.POINTER(C.c_uint64)]),
    "fa_fwd": (C.c_int, [C.POINTER(FaProblem), C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                         C.c_void_p, C.c_uint64, C.c_void_p]),
    "fa_fwd_lse": (C.c_int, [C.POINTER(FaProblem), C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                             C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p]),
    "fa_fwd_strided": (C.c_int, [C.POINTER(FaProblem), C.POINTER(FaStrides), C.c_void_p,
                                 C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                 C.c_uint64, C.c_void_p]),
    "fa_fwd_capture_count": (C.c_int, [C.POINTER(FaProblem), C.POINTER(C.c_uint64),
                                       C.POINTER(C.c_int32)]),
    "fa_fwd_capture": (C.c_int, [C.POINTER(FaProblem), C.c_void_p, C.c_void_p, C.c_void_p,
                                 C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p,
                                 C.c_uint64, C.c_void_p]),
    "fa_fwd_trace_count": (C.c_int, [C.POINTER(FaProblem), C.POINTER(C.c_uint64)]),
    "fa_fwd_trace": (C.c_int, [C.POINTER(FaProblem), C.c_void_p, C.c_void_p, C.c_void_p,
                               C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p, C.c_uint64,
                               C.c_void_p]),
    "fa_fwd_sync": (C.c_int, [C.POINTER(FaProblem), C.c_void_p, C.c_void_p, C.c_void_p,
                              C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p]),
    "fa_fwd_noalloc": (C.c_int, [C.POINTER(FaProblem), C.c_void_p, C.c_void_p, C.c_void_p,
                                 C.c_void_p, C.c_void_p]),
    "fa_fwd_split_count": (C.c_int, [C.POINTER(FaProblem), C.c_int32, C.c_int32,
                                     C.POINTER(C.c_int32)]),
    "fa_fwd_split_workspace_bytes": (C.c_int, [C.POINTER(FaProblem), C.c_int32,
                                               C.POINTER(C.c_uint64)]),
    "fa_fwd_split": (C.c_int, [C.POINTER(FaProblem), C.c_int32, C.POINTER(FaStrides), C.c_void_p,
                               C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                               C.c_uint64, C.c_void_p]),
    "fa_fwd_tile": (C.c_int, [C.POINTER(FaProblem), C.POINTER(C.c_int32), C.POINTER(C.c_int32)]),
    "fa_fwd_select": (C.c_int, [C.POINTER(FaProblem), C.POINTER(C.c_int32)]),
    "fa_kernel_count": (C.c_int, []),
    "fa_kernel_name": (C.c_char_p, [C.c_int32]),
    "fa_strerror": (C.c_char_p, [C.c_int]),
}


def load_library(path):
    """Open the shared library and attach the C signatures of every entry point."""
    lib = C.CDLL(str(path), mode=C.RTLD_LOCAL)
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return lib


@dataclass(frozen=True)
class AttentionConfig:
    """Launch configuration: accumulation variant, tile selector (0 = automatic),
    capture (debug) mode, which records every row's online-softmax
    statistics per key block (the reference config's ``capture`` flag,
    ``backends/cce_fa_nk_nz_vector_fp32_v5_sumpack/backend.py:27``), the
    attention mask (``FA_CAUSAL``; a row that sees no key gets O = 0 and
    lse = -inf), trace mode, which records per 256-row query tile where
    it ran and its clock stamps (the reference kernel's ``trace`` output),
    and the synchronous debug mode (``fa_fwd_sync``: poisoned staging
    buffers, no load/compute overlap; the reference's ``SYNCHRONOUS`` build
    flag), whose output must equal the production kernel's bit for bit.
    ``splits`` selects the key-split forward (``fa_fwd_split``): None (the
    default) runs one work item per query tile, 0 lets the library choose a
    split count, n >= 1 asks for n parts of every tile's key range (1 is the
    unsplit forward)."""
    acc: str = "fp32"
    kernel: int = 0
    capture: bool = False
    causal: str = "none"
    trace: bool = False
    sync: bool = False
    splits: "int | None" = None

    def __post_init__(self):
        if self.acc not in FA_ACC:
            raise ValueError(f"unknown accumulation variant {self.acc!r}")
        if not isinstance(self.kernel, int) or self.kernel < 0:
            raise ValueError("kernel selector must be a non-negative int")
        if not isinstance(self.capture, bool):
            raise ValueError("capture must be a bool")
        if self.causal not in FA_CAUSAL:
            raise ValueError(f"unknown causal mode {self.causal!r}")
        if not isinstance(self.trace, bool):
            raise ValueError("trace must be a bool")
        if not isinstance(self.sync, bool):
            raise ValueError("sync must be a bool")
        if self.trace + self.capture + self.sync > 1:
            raise ValueError("capture, trace and sync are separate kernels; pick one")
        if self.splits is not None:
            if not isinstance(self.splits, int) or isinstance(self.splits, bool) \
                    or not 0 <= self.splits <= 1024:
                raise ValueError("splits must be None or an int in 0..1024")
            if self.capture or self.trace or self.sync:
                raise ValueError("the key-split forward has no capture, trace or sync mode")


# Query rows per attention tile.
TILE_ROWS = 256


def query_tiles(batch, heads_q, heads_kv, seq_q):
    """Attention tiles of one launch, as the library lays them out: unpacked,
    ``batch * heads_q`` row sequences of ``seq_q`` query rows; packed, when
    that needs fewer 256-row tiles (grouped-query attention with few query
    rows), ``batch * heads_kv`` sequences of ``seq_q * group`` rows, the
    group's query heads position by position. Every row's result is the same
    either way. (One trace record per tile: ``fa_fwd_trace_count`` / 8.)"""
    def tiles(seqs, rows):
        return seqs * -(-rows // TILE_ROWS)

    plain = tiles(batch * heads_q, seq_q)
    group = heads_q // heads_kv
    if group <= 1 or seq_q * group >= 2 ** 30:
        return plain
    return min(plain, tiles(batch * heads_kv, seq_q * group))


def make_problem(q_shape, k_shape, scale, config):
    b, hq, nq, d = q_shape
    _, hkv, nk, _ = k_shape
    return FaProblem(b, hq, hkv, nq, nk, d, float(scale), FA_ACC[config.acc], config.kernel,
                     FA_CAUSAL[config.causal])


class Operator:
    """Callable ``(q, k, v) -> o`` over ``libfa_hip.so``."""

    def __init__(self, library, config=AttentionConfig()):
        self.config = config
        self.lib = load_library(library) if not isinstance(library, C.CDLL) else library
        self.workspace = None
        self.buffers = {}
        self.plans = {}          # (shapes, scale, device) -> (FaProblem, workspace bytes)
        self.tiles = {}          # (q shape, k shape) -> (rows, keys) granularity
        self.last = None

    def message(self, status):
        text = self.lib.fa_strerror(status)
        return text.decode() if text else "unknown status"

    def check(self, status, where):
        if status:
            raise RuntimeError(f"fa_fwd {where}: {status} ({self.message(status)})")

    def tile(self, q_shape, k_shape):
        """(query rows, keys) granularity of the kernel the library would use."""
        key = (tuple(q_shape), tuple(k_shape))
        if key not in self.tiles:
            prob = make_problem(q_shape, k_shape, 1.0, self.config)
            rows, keys = C.c_int32(), C.c_int32()
            self.check(self.lib.fa_fwd_tile(C.byref(prob), C.byref(rows), C.byref(keys)), "tile")
            self.tiles[key] = (rows.value, keys.value)
        return self.tiles[key]

    def kernel(self, q_shape, k_shape):
        """1-based tile configuration the library would launch (automatic choice resolved)."""
        prob = make_problem(q_shape, k_shape, 1.0, self.config)
        idx = C.c_int32()
        self.check(self.lib.fa_fwd_select(C.byref(prob), C.byref(idx)), "select")
        return idx.value

    def kernel_name(self, q_shape, k_shape):
        return self.lib.fa_kernel_name(self.kernel(q_shape, k_shape)).decode()

    def split_count(self, q_shape, k_shape, cus=0):
        """Key-range parts per query tile the key-split forward would run
        (``config.splits`` resolved; ``cus`` = 0: the current device)."""
        if self.config.splits is None:
            return 1
        prob = make_problem(q_shape, k_shape, 1.0, self.config)
        n = C.c_int32()
        self.check(self.lib.fa_fwd_split_count(C.byref(prob), self.config.splits, cus,
                                               C.byref(n)), "split")
        return n.value

    def validate(self, q, k, v):
        import torch

        if q.ndim != 4 or k.ndim != 4 or v.shape != k.shape:
            raise ValueError("Q/K/V must be [B,H,N,128]")
        b, h, nq, d = q.shape
        if min(q.shape) <= 0 or min(k.shape) <= 0 or k.shape[0] != b or d != 128 \
                or k.shape[3] != 128 or h % k.shape[1]:
            raise ValueError("invalid attention geometry")
        rows, keys = self.tile(q.shape, k.shape)
        if nq % rows or k.shape[2] % keys or max(nq, k.shape[2]) >= 2 ** 30:
            raise ValueError(f"unsupported query/key tail (Nq % {rows}, Nk % {keys})")
        for t in (q, k, v):
            if t.device.type != "cuda" or t.device != q.device or t.dtype != torch.float16:
                raise ValueError("Q/K/V must be FP16 on the same GPU")
            st = t.stride()
            if st[3] != 1 or any(x % 8 or x < 0 for x in st[:3]) or st[2] < 128 \
                    or t.data_ptr() % 16:
                raise ValueError("Q/K/V must be [B,H,N,128] views with a contiguous last "
                                 "dimension and 16-byte aligned rows")

    def buffers_for(self, q, k, lse=False):
        import torch

        key = (tuple(q.shape), tuple(k.shape), q.device, self.config, lse)
        if key not in self.buffers:
            if lse:
                self.buffers[key] = torch.empty(q.shape[:3], dtype=torch.float32, device=q.device)
            else:
                self.buffers[key] = torch.empty(q.shape, dtype=torch.float16, device=q.device)
        return self.buffers[key]

    # Capture buffers are for small debug inputs, as in the reference binding
    # (binding.py:40-42: at most 64 Mi FP32 values).
    CAPTURE_LIMIT = 64 * 1024 * 1024

    def stats_for(self, q, k, prob):
        import torch

        key = (tuple(q.shape), tuple(k.shape), q.device, self.config, "stats")
        if key not in self.buffers:
            count, block = C.c_uint64(), C.c_int32()
            self.check(self.lib.fa_fwd_capture_count(C.byref(prob), C.byref(count),
                                                     C.byref(block)), "capture")
            if count.value > self.CAPTURE_LIMIT:
                raise ValueError("debug capture is restricted to small inputs (at most 256 MiB)")
            nblk = count.value // (4 * q.shape[0] * q.shape[1] * q.shape[2])
            stats = torch.empty((4, nblk) + tuple(q.shape[:3]), dtype=torch.float32,
                                device=q.device)
            self.buffers[key] = (stats, block.value)
        return self.buffers[key]

    def trace_for(self, q, k, prob):
        import torch

        key = (tuple(q.shape), tuple(k.shape), q.device, self.config, "trace")
        if key not in self.buffers:
            count = C.c_uint64()
            self.check(self.lib.fa_fwd_trace_count(C.byref(prob), C.byref(count)), "trace")
            self.buffers[key] = torch.empty((count.value // TRACE_WORDS, TRACE_WORDS),
                                            dtype=torch.int64, device=q.device)
        return self.buffers[key]

    def __call__(self, q, k, v, scale=None, return_lse=False):
        """O (cached tensor), or (O, lse) with ``return_lse``: lse [B, Hq, Nq] FP32
        natural-log log-sum-exp of the scaled scores of each query row.

        With ``config.capture`` the call also fills ``self.last["stats"]``,
        FP32 [4, nblk, B, Hq, Nq]: per key block of ``self.last["block_keys"]``
        keys, each row's running max m (natural-log units), running sum l
        relative to m, rescale factor alpha and block sum z relative to m.
        With ``config.trace`` it fills ``self.last["trace"]``, int64
        [tiles, 8]: the per-query-tile records of ``fa_fwd_trace``."""
        import torch

        self.validate(q, k, v)
        scale = q.shape[3] ** -0.5 if scale is None else float(scale)
        if not (scale > 0 and math.isfinite(scale)):
            raise ValueError("scale must be finite and positive")
        splits = self.config.splits
        # The problem and its workspace size depend on the shapes, the scale
        # and (automatic split count) the device only: computed once each.
        plan_key = (tuple(q.shape), tuple(k.shape), scale, q.device)
        if plan_key not in self.plans:
            prob = make_problem(q.shape, k.shape, scale, self.config)
            size = C.c_uint64()
            if splits is None:
                self.check(self.lib.fa_fwd_workspace_bytes(C.byref(prob), C.byref(size)),
                           "prepare")
            else:
                with torch.cuda.device(q.device):
                    self.check(self.lib.fa_fwd_split_workspace_bytes(C.byref(prob), splits,
                                                                     C.byref(size)), "prepare")
            self.plans[plan_key] = (prob, size.value)
        prob, size = self.plans[plan_key]
        out = self.buffers_for(q, k)
        capture = self.config.capture
        lse = self.buffers_for(q, k, lse=True) if (return_lse or capture) else None
        stats, block = self.stats_for(q, k, prob) if capture else (None, 0)
        trace = self.trace_for(q, k, prob) if self.config.trace else None
        strided = not all(t.is_contiguous() for t in (q, k, v))
        if strided and (capture or trace is not None or self.config.sync):
            raise ValueError("capture, trace and sync modes need contiguous Q/K/V")
        with torch.cuda.device(q.device):
            need = max(size, 16)
            if self.workspace is None or self.workspace.device != q.device \
                    or self.workspace.numel() < need:
                self.workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
            stream = torch.cuda.current_stream(q.device)
            common = (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr())
            tail = (self.workspace.data_ptr(), self.workspace.numel(),
                    C.c_void_p(stream.cuda_stream))
            st = None
            if strided:
                st = FaStrides()
                for name, t in (("q", q), ("k", k), ("v", v), ("o", out)):
                    getattr(st, name)[:] = t.stride()[:3]
            if splits is not None:
                status = self.lib.fa_fwd_split(C.byref(prob), splits,
                                               C.byref(st) if st is not None else None, *common,
                                               lse.data_ptr() if lse is not None else None, *tail)
            elif strided:
                status = self.lib.fa_fwd_strided(C.byref(prob), C.byref(st), *common,
                                                 lse.data_ptr() if lse is not None else None,
                                                 *tail)
            elif capture:
                status = self.lib.fa_fwd_capture(C.byref(prob), *common, lse.data_ptr(),
                                                 stats.data_ptr(), stats.numel(), *tail)
            elif trace is not None:
                status = self.lib.fa_fwd_trace(C.byref(prob), *common, trace.data_ptr(),
                                               trace.numel(), *tail)
            elif self.config.sync:
                status = self.lib.fa_fwd_sync(C.byref(prob), *common,
                                              lse.data_ptr() if lse is not None else None, *tail)
            elif return_lse:
                status = self.lib.fa_fwd_lse(C.byref(prob), *common, lse.data_ptr(), *tail)
            else:
                status = self.lib.fa_fwd(C.byref(prob), *common, *tail)
            self.check(status, "launch")
            extra = tuple(t for t in (lse, stats, trace) if t is not None)
            for t in (q, k, v, out, self.workspace) + extra:
                t.record_stream(stream)
        self.last = {"output": out, "lse": lse, "stats": stats, "block_keys": block,
                     "trace": trace}
        return (out, lse) if return_lse else out
