"""MI355X flash-attention forward, FP32-accumulated O (the headline variant).

Hand-written gfx950 HIP kernel behind the C ABI of ``libfa_hip.so``
(``include/fa_hip.h``): FP16 MFMA for QK^T and PV, K/V blocks staged in LDS
and shared by every wave of the workgroup, online softmax in FP32 registers,
O accumulated in FP32 registers across all keys. Numerical counterpart of the
reference's ``cce_fa_nk_nz_vector_fp32_v5_sumpack``
(``backends/cce_fa_nk_nz_vector_fp32_v5_sumpack/backend.py:11-17``).
"""

from fa_amd.backends import hip_common
from fa_amd.harness.contract import Meta

META = Meta(
    name="hip_fa_fp32acc",
    type="hip",
    op_type="hip_fa_fp32acc_kernel",
    author="fa_amd",
    notes="gfx950 MFMA f16 QK/PV, LDS-shared K/V blocks, FP32 softmax, FP32 O in registers",
)

ACC = "fp32"


def operator(case):
    return hip_common.operator(ACC, case)


def adapt(case, canonical):
    return hip_common.adapt(case, canonical)
