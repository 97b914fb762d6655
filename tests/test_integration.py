"""The reference-side drop-in module ``integration/hip_fa/backend.py``.

It is written against the reference's plugin API (``from core.contract import
Meta``), so the tests load it with ``core.contract`` bound to this package's
identical ``fa_amd.harness.contract``. On the CPU: the ``fa_problem`` struct it
builds matches the C header field by field, the workspace phase succeeds for
every configuration, geometry errors raise ``ValueError``, and the module
text in INTEGRATION.md is the committed file verbatim. On the GPU: the
forward through the module matches the float64 oracle at c0 and at a ragged
shape, also when driven by the external driver.
"""

import ctypes as C
import importlib.util
import sys
import types
from pathlib import Path

import numpy as np
import pytest
import torch

from fa_amd import binding
from fa_amd.harness import contract
from fa_amd.problem.cases import CASES, Case

REPO = Path(__file__).resolve().parent.parent
MODULE = REPO / "integration" / "hip_fa" / "backend.py"


@pytest.fixture(scope="module")
def hip_fa(library_path):
    core = types.ModuleType("core")
    core.contract = contract
    saved = {n: sys.modules.get(n) for n in ("core", "core.contract")}
    sys.modules["core"], sys.modules["core.contract"] = core, contract
    try:
        spec = importlib.util.spec_from_file_location("backends.hip_fa.backend", MODULE)
        module = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(module)
    finally:
        for n, m in saved.items():
            if m is None:
                sys.modules.pop(n, None)
            else:
                sys.modules[n] = m
    mp = pytest.MonkeyPatch()
    mp.setenv(module.LIBRARY_ENV, library_path)
    module._lib = None
    yield module
    mp.undo()


def test_meta_follows_the_reference_contract(hip_fa):
    assert isinstance(hip_fa.META, contract.Meta)
    assert hip_fa.META.type == "external" and not hip_fa.META.is_reference
    for hook in ("build", "adapt", "call"):
        assert callable(getattr(hip_fa, hook))
    # Device kernels of both variants carry the directory name.
    assert hip_fa.META.op_type.startswith("hip_fa")


def test_struct_layout_equals_the_header(hip_fa):
    mine, lib = hip_fa.FaProblem, binding.FaProblem
    assert [f[0] for f in mine._fields_] == [f[0] for f in lib._fields_]
    assert [f[1] for f in mine._fields_] == [f[1] for f in lib._fields_]
    assert C.sizeof(mine) == C.sizeof(lib)
    for name, _ in mine._fields_:
        assert getattr(mine, name).offset == getattr(lib, name).offset, name


@pytest.mark.parametrize("index", range(len(CASES)))
def test_problem_fields_and_workspace_for_every_configuration(hip_fa, index):
    case = CASES[index]
    q = torch.empty(case.batch, case.heads_q, case.seq_len, case.dim, device="meta")
    k = torch.empty(case.batch, case.heads_kv, case.seq_len, case.dim, device="meta")
    p = hip_fa.problem(case, q, k)
    assert (p.batch, p.heads_q, p.heads_kv, p.seq_q, p.seq_k, p.dim) == \
        (case.batch, 12, 1, case.seq_len, case.seq_len, 128)
    assert p.scale == pytest.approx(case.scale, rel=1e-7)
    assert (p.acc, p.kernel, p.causal) == (hip_fa.ACC, 0, 0)
    size = C.c_uint64()
    assert hip_fa._library().fa_fwd_workspace_bytes(C.byref(p), C.byref(size)) == 0
    # 12 x N query rows per KV head: the V^T tile, whose workspace is V^T
    # (B * Hkv * N rows of 256 bytes) and the 256-byte tile counter.
    assert size.value == case.batch * case.heads_kv * case.seq_len * 128 * 2 + 256


def test_adapt_on_host_tensors_and_its_errors(hip_fa):
    case = Case(1, 300, 4, 2)
    x = {n: torch.zeros(s, dtype=torch.float16) for n, s in
         (("q", (1, 4, 300, 128)), ("k", (1, 2, 300, 128)), ("v", (1, 2, 300, 128)))}
    args = hip_fa.adapt(case, x)
    assert args["out"].shape == x["q"].shape and args["out"].dtype == torch.float16
    assert args["workspace"].numel() >= 2 * 2 * 384 * 256      # padded K and V copies
    bad = dict(x, q=x["q"].float())
    with pytest.raises(ValueError):
        hip_fa.adapt(case, bad)
    with pytest.raises(ValueError):
        hip_fa.adapt(case, dict(x, k=torch.zeros(1, 3, 300, 128, dtype=torch.float16),
                                v=torch.zeros(1, 3, 300, 128, dtype=torch.float16)))
    hip_fa.build(case)


def test_integration_doc_includes_the_module_verbatim():
    doc = (REPO / "INTEGRATION.md").read_text()
    assert MODULE.read_text() in doc


@pytest.mark.gpu
@pytest.mark.parametrize("case", [CASES[0], Case(1, 1000, 12, 1)], ids=lambda c: c.name)
def test_forward_through_the_module_matches_the_oracle(hip_fa, case):
    from fa_amd.harness import drivers
    from fa_amd.problem.canonical import build_canonical
    from oracle.attention import attention_f64

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    print(f"case integration/hip_fa {case.name}", flush=True)
    cpu = build_canonical(case, seed=0)
    dev = {n: t.to("cuda") for n, t in cpu.items()}
    exact = attention_f64(cpu["q"], cpu["k"], cpu["v"])
    out = hip_fa.call(hip_fa.adapt(case, dev))
    torch.cuda.synchronize()
    err = float(np.abs(out.float().cpu().numpy() - exact).max())
    print(f"  max_abs_err={err:.3e}", flush=True)
    assert err <= 2e-3
    # The reference's external driver contract, run by this harness's copy of it.
    forward = drivers.driver("external").prepare(hip_fa, case)(dev)
    again = forward()
    torch.cuda.synchronize()
    assert torch.equal(again, out)
