"""Canonical flash-attention inputs: a pure function of the Case and the seed.

Every backend consumes the same canonical tensors, so their outputs compare
directly. Mirrors ``problem/canonical.py:18-28`` of the reference (seeded FP16
``randn`` drawn in the order q, k, v), with one deliberate difference: the
reference draws on the NPU's generator, whose stream is not reproducible on
other hardware, so the draw here happens on a CPU ``torch.Generator`` and the
finished tensors are copied to the device. The CPU oracle and the GPU kernels
therefore see bit-identical inputs.

Shapes (non-causal full attention, GQA via heads_q / heads_kv):
  q  [batch, heads_q,  seq_len, dim]  float16
  k  [batch, heads_kv, seq_len, dim]  float16
  v  [batch, heads_kv, seq_len, dim]  float16

``stress`` cases (see ``fa_amd.problem.cases``) draw the same three tensors in
the same order, then scale q and k by 3 in FP16, then draw one ``randperm``
over the ``batch * heads_kv * seq_len`` rows of v and multiply the first 5% of
that permutation's rows by 8.
"""

import torch

STRESS_QK_SCALE = 3.0
STRESS_V_FRACTION = 0.05
STRESS_V_SCALE = 8.0


def stress_row_count(case) -> int:
    return int(round(STRESS_V_FRACTION * case.batch * case.heads_kv * case.seq_len))


def build_canonical(case, seed: int = 0, device=None) -> dict:
    """Draw q, k, v for ``case`` on the CPU and move them to ``device``.

    ``device=None`` keeps the tensors on the CPU.
    """
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)

    def rand(*shape):
        return torch.randn(shape, generator=g, dtype=torch.float16)

    q = rand(case.batch, case.heads_q, case.seq_len, case.dim)
    k = rand(case.batch, case.heads_kv, case.seq_len, case.dim)
    v = rand(case.batch, case.heads_kv, case.seq_len, case.dim)
    if case.dist == "stress":
        q.mul_(STRESS_QK_SCALE)
        k.mul_(STRESS_QK_SCALE)
        rows = case.batch * case.heads_kv * case.seq_len
        chosen = torch.randperm(rows, generator=g)[: stress_row_count(case)]
        v.view(rows, case.dim)[chosen] *= STRESS_V_SCALE
    out = {"q": q, "k": k, "v": v}
    if device is not None:
        out = {name: t.to(device) for name, t in out.items()}
    return out
