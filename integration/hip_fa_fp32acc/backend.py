"""hip_fa_fp32acc -- the MI355X flash-attention forward as a platelett/fa backend.

Drop-in backend module for the reference harness: copy this directory to
``backends/hip_fa_fp32acc/`` of platelett/fa and point ``FA_HIP_LIBRARY`` at a
built ``libfa_hip.so`` (or place the library beside this file). It is an
``external`` backend (``core/drivers/external.py:23-26`` of the reference
drives it unchanged): ``adapt`` sizes the workspace through
``fa_fwd_workspace_bytes`` and allocates the output and workspace once per
case, ``call`` enqueues ``fa_fwd`` on the current torch stream and returns the
same output tensor every time, as the reference's own operator bindings do
(``backends/cce_fa_nk_nz_vector_fp32_v5_sumpack/binding.py:34-85``). Geometry
errors raise ``ValueError``, a failed launch ``RuntimeError``.

This module is the FP32-accumulated variant (the reference's FP32-O backend,
``backends/cce_fa_nk_nz_vector_fp32_v5_sumpack``). Its FP16-accumulated
sibling ``backends/hip_fa_fp16acc/`` (the reference's FP16-O backend,
``backends/cce_fa_nqkq_nz_resident_v13_q768_pool_i4_p128``) reuses the library
loader and the three hooks below with ``acc=1``.

The library's C ABI is declared in ``include/fa_hip.h`` of fa_amd; only three
of its entry points are needed here. Its device kernels are named
``hip_fa_fp32acc_kernel<...>`` / ``hip_fa_fp16acc_kernel<...>``: each contains
its own backend's directory name and not the other's, so the reference
profiler's name rule (``core/profiler.py:14-25``) attributes every attention
kernel to the backend that launched it.
"""

import ctypes as C
import os

from core.contract import Meta

META = Meta(
    name="hip_fa_fp32acc",
    type="external",
    op_type="hip_fa_fp32acc_kernel",
    author="fa_amd",
    notes="MI355X (gfx950) HIP flash-attention forward over libfa_hip.so; "
          "FP16 MFMA QK/PV, FP32 online softmax, FP32-accumulated O.",
)

# Accumulation variant (enum fa_acc): 0 = FP32-accumulated O (this backend),
# 1 = FP16-accumulated O (backends/hip_fa_fp16acc).
ACC = 0

LIBRARY_ENV = "FA_HIP_LIBRARY"


class FaProblem(C.Structure):
    """``fa_problem`` of include/fa_hip.h, field for field."""
    _fields_ = [
        ("batch", C.c_int64),
        ("heads_q", C.c_int64),
        ("heads_kv", C.c_int64),
        ("seq_q", C.c_int64),
        ("seq_k", C.c_int64),
        ("dim", C.c_int64),
        ("scale", C.c_float),
        ("acc", C.c_int32),
        ("kernel", C.c_int32),     # 0 = automatic tile choice
        ("causal", C.c_int32),     # 0 = full attention, the harness's only mode
    ]


_lib = None


def library_path():
    return os.environ.get(LIBRARY_ENV) or os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                       "libfa_hip.so")


def _library():
    global _lib
    if _lib is None:
        lib = C.CDLL(library_path(), mode=C.RTLD_LOCAL)
        lib.fa_fwd_workspace_bytes.restype = C.c_int
        lib.fa_fwd_workspace_bytes.argtypes = [C.POINTER(FaProblem), C.POINTER(C.c_uint64)]
        lib.fa_fwd.restype = C.c_int
        lib.fa_fwd.argtypes = [C.POINTER(FaProblem), C.c_void_p, C.c_void_p, C.c_void_p,
                               C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p]
        lib.fa_strerror.restype = C.c_char_p
        lib.fa_strerror.argtypes = [C.c_int]
        _lib = lib
    return _lib


def _message(status):
    text = _library().fa_strerror(status)
    return text.decode() if text else "unknown status"


def problem(case, q, k, acc=ACC):
    """The ``fa_problem`` of one forward over canonical q [B,Hq,N,128], k [B,Hkv,N,128]."""
    return FaProblem(batch=q.shape[0], heads_q=q.shape[1], heads_kv=k.shape[1],
                     seq_q=q.shape[2], seq_k=k.shape[2], dim=q.shape[3],
                     scale=case.scale, acc=acc, kernel=0, causal=0)


def build(case):
    """CPU-safe and idempotent: the prebuilt library must be where it is looked for."""
    if not os.path.isfile(library_path()):
        raise FileNotFoundError(f"libfa_hip.so not found at {library_path()} "
                                f"(set {LIBRARY_ENV})")


def adapt(case, canonical, acc=ACC):
    import torch

    q, k, v = canonical["q"], canonical["k"], canonical["v"]
    for t in (q, k, v):
        if t.dtype != torch.float16 or t.dim() != 4 or not t.is_contiguous() \
                or t.device != q.device:
            raise ValueError("hip_fa needs contiguous FP16 [B,H,N,128] q/k/v on one device")
    if k.shape != v.shape or k.shape[0] != q.shape[0] or q.shape[3] != 128 \
            or k.shape[3] != 128 or q.shape[1] % k.shape[1]:
        raise ValueError("invalid attention geometry for hip_fa")
    p = problem(case, q, k, acc)
    size = C.c_uint64()
    status = _library().fa_fwd_workspace_bytes(C.byref(p), C.byref(size))
    if status:
        raise ValueError(f"fa_fwd_workspace_bytes: {status} ({_message(status)})")
    out = torch.empty_like(q)
    workspace = torch.empty(max(size.value, 16), dtype=torch.uint8, device=q.device)
    return {"problem": p, "q": q, "k": k, "v": v, "out": out, "workspace": workspace}


def call(op_args):
    import torch

    a = op_args
    with torch.cuda.device(a["q"].device):     # the library works on the current device
        stream = torch.cuda.current_stream(a["q"].device)
        status = _library().fa_fwd(C.byref(a["problem"]), a["q"].data_ptr(), a["k"].data_ptr(),
                                   a["v"].data_ptr(), a["out"].data_ptr(),
                                   a["workspace"].data_ptr(), a["workspace"].numel(),
                                   C.c_void_p(stream.cuda_stream))
    if status:
        raise RuntimeError(f"fa_fwd launch: {status} ({_message(status)})")
    return a["out"]
