"""hip_fa_fp16acc -- the FP16-accumulated MI355X forward as a platelett/fa backend.

The second drop-in backend, beside ``backends/hip_fa_fp32acc/``: the
reference ships its FP32-O and FP16-O kernels as two backend directories
(``backends/cce_fa_nk_nz_vector_fp32_v5_sumpack``,
``backends/cce_fa_nqkq_nz_resident_v13_q768_pool_i4_p128``), and so does this
library. Copy this directory to ``backends/hip_fa_fp16acc/`` next to
``backends/hip_fa_fp32acc/``, whose library loader (``FA_HIP_LIBRARY``, the
same ``libfa_hip.so``) and ``external`` hooks it reuses with the
FP16-accumulated variant selected (``fa_problem.acc = 1``: O rounded to FP16
at every 512-key packet, as the reference's FP16-O merge does). Its kernels
are named ``hip_fa_fp16acc_kernel<...>``, so the reference profiler's name
rule (``core/profiler.py:14-25``) attributes them to this directory.
"""

from backends.hip_fa_fp32acc import backend as _fa
from core.contract import Meta

META = Meta(
    name="hip_fa_fp16acc",
    type="external",
    op_type="hip_fa_fp16acc_kernel",
    author="fa_amd",
    notes="MI355X (gfx950) HIP flash-attention forward over libfa_hip.so; "
          "FP16 MFMA QK/PV, FP32 online softmax, FP16-accumulated O (rounded every 512 keys).",
)

# Accumulation variant (enum fa_acc): 1 = FP16-accumulated O.
ACC = 1

LIBRARY_ENV = _fa.LIBRARY_ENV
FaProblem = _fa.FaProblem


def problem(case, q, k):
    return _fa.problem(case, q, k, acc=ACC)


def build(case):
    _fa.build(case)


def adapt(case, canonical):
    return _fa.adapt(case, canonical, acc=ACC)


def call(op_args):
    return _fa.call(op_args)
