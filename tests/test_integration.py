"""The reference-side drop-in modules ``integration/hip_fa_fp32acc/backend.py``
and ``integration/hip_fa_fp16acc/backend.py``.

They are written against the reference's plugin API (``from core.contract
import Meta``; the FP16 module imports its sibling as
``backends.hip_fa_fp32acc.backend``, as the reference registry imports
backend modules), so the tests load them under those names with
``core.contract`` bound to this package's identical
``fa_amd.harness.contract``. On the CPU: the ``fa_problem`` struct matches
the C header field by field, the workspace phase succeeds for every
configuration, geometry errors raise ``ValueError``, the reference
profiler's kernel-name rule attributes each variant's kernels to its own
directory, and the module texts in INTEGRATION.md are the committed files
verbatim. On the GPU: the forward through either module matches the float64
oracle at c0 and at a ragged shape, also when driven by the external driver.
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
MODULES = {name: REPO / "integration" / name / "backend.py"
           for name in ("hip_fa_fp32acc", "hip_fa_fp16acc")}
MODULE = MODULES["hip_fa_fp32acc"]
# North-star bars on the FP16 output: FP32- and FP16-accumulated O.
BARS = {"hip_fa_fp32acc": 2e-3, "hip_fa_fp16acc": 1e-2}


@pytest.fixture(scope="module")
def modules(library_path):
    """Both backend modules, imported as the reference registry would."""
    core = types.ModuleType("core")
    core.contract = contract
    pkg = types.ModuleType("backends")
    pkg.__path__ = []
    names = ["core", "core.contract", "backends"] + \
        [f"backends.{n}{s}" for n in MODULES for s in ("", ".backend")]
    saved = {n: sys.modules.get(n) for n in names}
    sys.modules.update({"core": core, "core.contract": contract, "backends": pkg})
    loaded = {}
    try:
        for name, path in MODULES.items():         # the FP32 module first: the FP16 one imports it
            sub = types.ModuleType(f"backends.{name}")
            sub.__path__ = []
            sys.modules[f"backends.{name}"] = sub
            spec = importlib.util.spec_from_file_location(f"backends.{name}.backend", path)
            module = importlib.util.module_from_spec(spec)
            sys.modules[spec.name] = module
            spec.loader.exec_module(module)
            sub.backend = module
            loaded[name] = module
    finally:
        for n, m in saved.items():
            if m is None:
                sys.modules.pop(n, None)
            else:
                sys.modules[n] = m
    mp = pytest.MonkeyPatch()
    mp.setenv(loaded["hip_fa_fp32acc"].LIBRARY_ENV, library_path)
    loaded["hip_fa_fp32acc"]._lib = None
    yield loaded
    mp.undo()


@pytest.fixture(scope="module")
def hip_fa(modules):
    return modules["hip_fa_fp32acc"]


@pytest.mark.parametrize("name", list(MODULES))
def test_meta_follows_the_reference_contract(modules, name):
    mod = modules[name]
    assert isinstance(mod.META, contract.Meta)
    assert mod.META.type == "external" and not mod.META.is_reference
    assert mod.META.name == name and mod.META.op_type == f"{name}_kernel"
    for hook in ("build", "adapt", "call"):
        assert callable(getattr(mod, hook))
    assert mod.ACC == {"hip_fa_fp32acc": 0, "hip_fa_fp16acc": 1}[name]
    # One loader for both: the FP16 module reuses its sibling's library.
    assert mod.LIBRARY_ENV == modules["hip_fa_fp32acc"].LIBRARY_ENV


def test_profiler_name_rule_attributes_each_variant_to_its_directory(modules):
    """The reference profiler's rule (``core/profiler.py:14-25``: exact
    symbol, else directory name or op_type substring), with both backend
    directories registered, sends every attention kernel of the library to
    the backend that launched it and leaves the prep kernels unclaimed."""
    from fa_amd.harness.timing import KernelOwners

    owners = KernelOwners(list(MODULES), op_types={n: m.META.op_type for n, m in modules.items()})
    for name in MODULES:
        for targs in ("128, 2, 0, false, false", "64, 3, 4, true, false", "128, 2, 0, true, true"):
            demangled = (f"void (anonymous namespace)::{name}_kernel<{targs}>"
                         "((anonymous namespace)::FaArgs)")
            assert owners.owner(demangled) == name
        mangled = f"_ZN12_GLOBAL__N_121{name}_kernelILi128ELi2ELi0ELb0ELb0EEEvNS_6FaArgsE"
        assert owners.owner(mangled) == name
    for other in ("_ZN12_GLOBAL__N_114fa_prep_kernelEPKDF16_S1_PDF16_S2_iiiNS_7StridesES3_Pi",
                  "_ZN12_GLOBAL__N_115fa_merge_kernelEPKfS1_PDF16_PfiliiNS_7StridesE"):
        assert owners.owner(other) is None


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


def test_fp16_module_sets_the_fp16_accumulator(modules):
    case = CASES[2]
    q = torch.empty(case.batch, case.heads_q, case.seq_len, case.dim, device="meta")
    k = torch.empty(case.batch, case.heads_kv, case.seq_len, case.dim, device="meta")
    p16 = modules["hip_fa_fp16acc"].problem(case, q, k)
    p32 = modules["hip_fa_fp32acc"].problem(case, q, k)
    assert (p16.acc, p32.acc) == (1, 0)
    x = {n: torch.zeros(s, dtype=torch.float16) for n, s in
         (("q", (1, 4, 300, 128)), ("k", (1, 2, 300, 128)), ("v", (1, 2, 300, 128)))}
    assert modules["hip_fa_fp16acc"].adapt(Case(1, 300, 4, 2), x)["problem"].acc == 1
    modules["hip_fa_fp16acc"].build(case)


@pytest.mark.parametrize("name", list(MODULES))
def test_integration_doc_includes_the_module_verbatim(name):
    doc = (REPO / "INTEGRATION.md").read_text()
    assert MODULES[name].read_text() in doc


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(MODULES))
@pytest.mark.parametrize("case", [CASES[0], Case(1, 1000, 12, 1)], ids=lambda c: c.name)
def test_forward_through_the_module_matches_the_oracle(modules, name, case):
    from fa_amd.harness import drivers
    from fa_amd.problem.canonical import build_canonical
    from oracle.attention import attention_f64

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    mod = modules[name]
    print(f"case integration/{name} {case.name}", flush=True)
    cpu = build_canonical(case, seed=0)
    dev = {n: t.to("cuda") for n, t in cpu.items()}
    exact = attention_f64(cpu["q"], cpu["k"], cpu["v"])
    out = mod.call(mod.adapt(case, dev))
    torch.cuda.synchronize()
    err = float(np.abs(out.float().cpu().numpy() - exact).max())
    print(f"  max_abs_err={err:.3e}", flush=True)
    assert err <= BARS[name]
    # The reference's external driver contract, run by this harness's copy of it.
    forward = drivers.driver("external").prepare(mod, case)(dev)
    again = forward()
    torch.cuda.synchronize()
    assert torch.equal(again, out)
