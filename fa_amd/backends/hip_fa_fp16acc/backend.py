"""MI355X flash-attention forward, FP16-accumulated O.

Hand-written gfx950 HIP kernel behind the C ABI of ``libfa_hip.so``
(``include/fa_hip.h``): FP16 MFMA for QK^T and PV, K/V blocks staged in LDS
and shared by every wave of the workgroup, online softmax in FP32 registers,
each block's PV product rounded to FP16 and merged into an FP16 O
accumulator (O = alpha*O + PV16). Numerical counterpart of the
reference's ``cce_fa_nqkq_nz_resident_v13_q768_pool_i4_p128``
(``backends/cce_fa_nqkq_nz_resident_v13_q768_pool_i4_p128/backend.py:12-18``).
"""

from fa_amd.backends import hip_common
from fa_amd.harness.contract import Meta

META = Meta(
    name="hip_fa_fp16acc",
    type="hip",
    op_type="hip_fa_fp16acc_kernel",
    author="fa_amd",
    notes="gfx950 MFMA f16 QK/PV, LDS-shared K/V blocks, FP32 softmax, FP16 O in registers",
)

ACC = "fp16"


def operator(case):
    return hip_common.operator(ACC, case)


def adapt(case, canonical):
    return hip_common.adapt(case, canonical)
