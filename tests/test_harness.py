"""Host-only tests of the harness: catalog, drivers, report, kernel attribution, CLI.

Everything runs on the CPU. Fake backend modules are plain namespaces;
device work is replaced by CPU tensors and patched timing, so what is tested
is the protocol: what is loaded when, what is compared with what, what a
failure turns into.
"""

import csv
from types import SimpleNamespace
from unittest.mock import Mock, patch

import pytest
import torch

from fa_amd.harness import drivers, report, timing
from fa_amd.harness.catalog import Backend, Catalog
from fa_amd.harness.contract import KernelNameError, Meta
from fa_amd.problem.cases import CASES, Case


def fake(name, kind="external", ref=False, diagnostic=False, **hooks):
    module = SimpleNamespace(__name__=f"fake.{name}",
                             META=Meta(name=name, type=kind, op_type=f"{name}_op",
                                       is_reference=ref, diagnostic=diagnostic),
                             **hooks)
    return Backend(name, module)


def catalog_of(*entries):
    return Catalog({e.name: e for e in entries})


# --------------------------------------------------------------------------- catalog

def test_package_catalog_has_three_backends_and_one_reference():
    cat = Catalog.default(rescan=True)
    assert sorted(cat.names()) == ["hip_fa_fp16acc", "hip_fa_fp32acc", "torch_ref"]
    assert cat.reference.name == "torch_ref"
    for n in cat.names():
        entry = cat[n]
        assert cat.name_of(entry.module) == n
        assert entry.driver.kind == entry.meta.type
    for n in ("hip_fa_fp32acc", "hip_fa_fp16acc"):
        assert cat[n].meta.type == "hip" and cat[n].meta.op_type == f"{n}_kernel"


@pytest.mark.parametrize("refs", [0, 2])
def test_catalog_needs_exactly_one_reference(refs):
    entries = [fake(f"b{i}", ref=i < refs) for i in range(3)]
    with pytest.raises(ValueError, match="exactly one reference"):
        catalog_of(*entries)


def test_unknown_backend_type_and_name():
    cat = catalog_of(fake("r", ref=True), fake("t", kind="tilelang"))
    with pytest.raises(drivers.UnknownBackendType):
        cat["t"].driver
    with pytest.raises(KeyError, match="no backend 'x'"):
        cat["x"]


def test_diagnostic_backends_are_listed_but_never_checked():
    cat = catalog_of(fake("r", ref=True), fake("probe", diagnostic=True))
    assert cat.names() == ["r"]
    assert cat.names(include_diagnostic=True) == ["r", "probe"]
    with pytest.raises(ValueError, match="diagnostic"):
        cat.attention("probe")


def test_name_of_rejects_unknown_or_doubly_registered_modules():
    r, b = fake("r", ref=True), fake("b")
    cat = catalog_of(r, b, Backend("alias", b.module))
    with pytest.raises(ValueError):
        cat.name_of(b.module)
    assert cat.name_of(r.module) == "r"
    with pytest.raises(ValueError):
        cat.name_of(SimpleNamespace(__name__="stranger"))


# --------------------------------------------------------------------------- drivers

def test_external_driver_adapts_late_and_calls_every_time():
    events = []
    module = SimpleNamespace(__name__="m",
                             build=lambda case: events.append(("build", case)),
                             adapt=lambda case, inputs: events.append(("adapt", inputs)) or "args",
                             call=lambda args: events.append(("call", args)) or "out")
    d = drivers.driver("external")
    assert d.needs_build(module)
    bind = d.prepare(module, "case")
    assert events == [("build", "case")]
    forward = bind("inputs")
    assert events[-1] == ("adapt", "inputs")
    assert forward() == "out" and forward() == "out"
    assert events.count(("call", "args")) == 2


def test_external_driver_without_build_and_with_a_broken_one():
    d = drivers.driver("external")
    plain = SimpleNamespace(__name__="m", adapt=Mock(return_value=1), call=Mock(return_value=2))
    assert not d.needs_build(plain)
    assert d.prepare(plain, "case")("inputs")() == 2
    plain.call.assert_called_once_with(1)
    broken = SimpleNamespace(__name__="m", build="not callable", adapt=Mock(), call=Mock())
    with pytest.raises(TypeError):
        d.prepare(broken, "case")


def test_hip_driver_loads_before_inputs_and_checks_hooks():
    d = drivers.driver("hip")
    forward = Mock(return_value="o")
    module = SimpleNamespace(__name__="m", operator=Mock(return_value=forward),
                             adapt=Mock(return_value=("q", "k", "v")))
    with patch("fa_amd.build.build") as build:
        bind = d.prepare(module, "case")
        build.assert_called_once()
    module.operator.assert_called_once_with("case")
    module.adapt.assert_not_called()
    call = bind("canonical")
    module.adapt.assert_called_once_with("case", "canonical")
    assert call() == "o"
    forward.assert_called_once_with("q", "k", "v")

    with patch("fa_amd.build.build"):
        with pytest.raises(TypeError, match="missing operator"):
            d.prepare(SimpleNamespace(__name__="m", adapt=Mock()), "case")
        module.operator.return_value = None
        with pytest.raises(TypeError, match="callable"):
            d.prepare(module, "case")
        module.operator.return_value = forward
        module.adapt.return_value = {"q": 1}
        with pytest.raises(TypeError, match="tuple"):
            d.prepare(module, "case")("canonical")


def test_hip_backends_load_the_built_library_only():
    from fa_amd import build
    from fa_amd.backends import hip_common

    with patch.object(build, "LIBRARY", build.LIBDIR / "missing.so"):
        with pytest.raises(FileNotFoundError):
            hip_common.operator("fp32", CASES[0])


# --------------------------------------------------------------------------- reference backend

def test_reference_backend_is_the_fp32_formula():
    from fa_amd.backends.torch_ref import backend

    g = torch.Generator().manual_seed(3)
    q = torch.randn(2, 6, 40, 128, generator=g).half()
    k = torch.randn(2, 3, 72, 128, generator=g).half()
    v = torch.randn(2, 3, 72, 128, generator=g).half()
    case = SimpleNamespace(heads_q=6, scale=0.1)
    out = backend.call(backend.adapt(case, {"q": q, "k": k, "v": v}))
    ke, ve = k.float().repeat_interleave(2, 1), v.float().repeat_interleave(2, 1)
    want = torch.softmax(q.float() @ ke.transpose(-1, -2) * 0.1, -1) @ ve
    assert out.dtype == torch.float16 and out.shape == q.shape
    assert float((out.float() - want).abs().max()) <= 2 ** -10
    small = backend.attention(q, k, v, 0.1, chunk_elems=72 * 7)     # ragged row chunks
    assert float((small.float() - want).abs().max()) <= 2 ** -10


# --------------------------------------------------------------------------- report

def run_report(entries, case=CASES[0], **kw):
    cat = catalog_of(*entries)
    inputs = {"q": torch.ones(1)}
    with patch("fa_amd.problem.canonical.build_canonical", return_value=inputs) as draw, \
            patch.object(torch.cuda, "synchronize"), \
            patch.object(timing, "device_us", return_value=50.0):
        rows = report.run_case(cat, case, [e.name for e in entries], device="cpu",
                               log=lambda *_: None, **kw)
    return rows, draw


def test_report_prepares_everything_before_drawing_inputs():
    events = []

    def module(name, out):
        return SimpleNamespace(
            __name__=name,
            build=lambda case: events.append(f"build {name}"),
            adapt=lambda case, inputs: events.append(f"adapt {name}") or None,
            call=lambda args: out)

    ref = Backend("ref", module("ref", torch.zeros(4)))
    ref.module.META = Meta("ref", "external", "ref", is_reference=True)
    mine = Backend("mine", module("mine", torch.full((4,), 0.005)))
    mine.module.META = Meta("mine", "external", "mine")

    def draw(*a, **k):
        events.append("inputs")
        return {}

    cat = catalog_of(ref, mine)
    with patch("fa_amd.problem.canonical.build_canonical", side_effect=draw), \
            patch.object(torch.cuda, "synchronize"), \
            patch.object(timing, "device_us", side_effect=[100.0, 25.0]):
        rows = report.run_case(cat, CASES[0], ["mine"], device="cpu", log=lambda *_: None)
    assert events == ["build ref", "build mine", "inputs", "adapt ref", "adapt mine"]
    by = {r.backend: r for r in rows}
    assert by["ref"].check == "ref" and by["mine"].check == "PASS"
    assert by["mine"].max_diff == pytest.approx(0.005)
    assert by["mine"].vs_ref == pytest.approx(0.25)
    cells = by["mine"].cells()
    assert cells[:6] == ["B1_S4096_Q12_KV1_D128", "mine", "", "25.00", "25.0%", "PASS"]
    assert float(cells[7]) == pytest.approx(CASES[0].flops / 25e-6 / 1e12, rel=1e-3)


def test_report_fails_a_wrong_backend_and_skips_a_broken_one():
    ref = fake("ref", ref=True, adapt=Mock(), call=Mock(return_value=torch.zeros(8)))
    wrong = fake("wrong", adapt=Mock(), call=Mock(return_value=torch.full((8,), 0.5)))
    broken = fake("broken", build=Mock(side_effect=OSError("no library")), adapt=Mock(),
                  call=Mock())
    crashing = fake("crashing", adapt=Mock(), call=Mock(side_effect=RuntimeError("launch")))
    rows, _ = run_report([ref, wrong, broken, crashing])
    by = {r.backend: r for r in rows}
    assert by["wrong"].check == "FAIL" and by["wrong"].max_diff == pytest.approx(0.5)
    assert by["broken"].check == "ERR" and by["broken"].avg_us is None
    assert by["crashing"].check == "ERR"
    assert by["broken"].cells()[3] == "N/A"
    broken.module.call.assert_not_called()


def test_report_never_swallows_kernel_name_errors():
    ref = fake("ref", ref=True, adapt=Mock(), call=Mock(return_value=torch.zeros(1)))
    bad = fake("bad", adapt=Mock(), call=Mock(side_effect=KernelNameError("unnamed kernel")))
    with pytest.raises(KernelNameError):
        run_report([ref, bad])


def test_check_backend_compares_with_the_reference():
    ref = fake("ref", ref=True, adapt=Mock(), call=Mock(return_value=torch.zeros(3)))
    close = fake("close", adapt=Mock(), call=Mock(return_value=torch.tensor([0., 0.004, 0.])))
    cat = catalog_of(ref, close)
    with patch("fa_amd.problem.canonical.build_canonical", return_value={}):
        assert report.check_backend(cat, "close", CASES[0], device="cpu") == (True, pytest.approx(0.004))
        assert report.check_backend(cat, "ref", CASES[0], device="cpu") == (True, 0.0)
        passed, diff = report.check_backend(cat, "close", CASES[0], device="cpu",
                                            tol=report.Tolerance(1e-3, 0.0))
    assert not passed and diff == pytest.approx(0.004)
    line = report.check_line(CASES[3], "close", False, 0.004)
    assert line == ("CHECK B2_S131072_Q12_KV1_D128 backend=close FAIL max_abs_diff=0.00400 "
                    "(atol=0.01, rtol=0.01)")


def test_report_csv_has_the_reference_columns_first(tmp_path):
    rows = [report.Row("c", "b", False, 10.0, 0.5, "PASS", 1e-4, 3.0)]
    path = tmp_path / "r.csv"
    report.write_csv(rows, path)
    head, body = list(csv.reader(open(path)))
    assert head[:7] == ["Case", "Backend", "Ref", "Avg_us", "vs_ref", "Check", "MaxDiff"]
    assert body == ["c", "b", "", "10.00", "50.0%", "PASS", "0.00010", "3.0", "0.1%"]


# --------------------------------------------------------------------------- kernel attribution

def test_declared_symbols_match_exactly_and_only_exactly():
    owners = KernelOwnersCase.owners()
    for kernel, backend in KernelOwnersCase.EXPECTED.items():
        assert owners.owner(kernel) == backend, kernel


class KernelOwnersCase:
    EXPECTED = {
        "attn_kernel": "attn",                        # default exact symbol <dir>_kernel
        "attn_v2_kernel": "attn_v2",                  # exact beats attn's substring
        "fast_main": "fast",                          # declared symbol
        "fast_main_v2": None,                         # declared backends never match loosely
        "fast_kernel": None,                          # ... not even by the default symbol
        "FlashAttentionScore_1": "vendor",            # op_type substring
        "xx_vendor_yy": "vendor",                     # directory-name substring
        "attn_kernel_tail": "attn",                   # substring for undeclared backends
        "unrelated": None,
    }

    @staticmethod
    def owners():
        return timing.KernelOwners(["attn", "attn_v2", "fast", "vendor"],
                                   op_types={"vendor": "FlashAttentionScore", "fast": "main"},
                                   symbols={"fast": "fast_main"})


def test_hip_kernels_are_attributed_to_their_backend(tmp_path):
    cat = Catalog.default()
    names = ["hip_fa_fp32acc", "hip_fa_fp16acc", "torch_ref"]
    owners = timing.KernelOwners(names, op_types={n: cat[n].meta.op_type for n in names})
    mangled = "_ZN12_GLOBAL__N_121hip_fa_fp32acc_kernelILi1ELi2ELi1ELi128ELi2ELb0EEEvNS_6FaArgsE"
    assert owners.owner(mangled) == "hip_fa_fp32acc"
    assert owners.owner(mangled.replace("fp32acc", "fp16acc")) == "hip_fa_fp16acc"
    assert owners.owner("_ZN12_GLOBAL__N_114fa_prep_kernelEPKDF16_") is None
    trace = tmp_path / "kernel_trace.csv"
    trace.write_text('"Kernel_Name","Start_Timestamp","End_Timestamp"\n'
                     f'"{mangled}",1000,3000\n"{mangled}",5000,9000\n"other",0,100\n')
    assert owners.average_us(trace) == {"hip_fa_fp32acc": 3.0, "hip_fa_fp16acc": None,
                                        "torch_ref": None}


def test_kernels_command_reports_per_backend_kernel_time(tmp_path, capsys):
    """``python -m fa_amd.harness kernels <dir>``: each backend's mean kernel
    duration from a rocprofv3 CSV trace (warmup dispatches skipped), the prep
    kernel listed as unowned."""
    from fa_amd.harness.__main__ import main

    k32 = "_ZN12_GLOBAL__N_121hip_fa_fp32acc_kernelILi128ELi2ELi0ELb0ELb0EEEvNS_6FaArgsE"
    k16 = k32.replace("fp32acc", "fp16acc")
    prep = "_ZN12_GLOBAL__N_114fa_prep_kernelEPKDF16_"
    folder = tmp_path / "run"
    folder.mkdir()
    rows = [(k32, 0, 9000), (prep, 9000, 9100), (k32, 10000, 12000), (k32, 20000, 24000),
            (k16, 30000, 39000), (k16, 40000, 45000), (prep, 45000, 45300)]
    with open(folder / "run_kernel_trace.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writerows(rows)
    cat = Catalog.default()
    names = ["hip_fa_fp32acc", "hip_fa_fp16acc", "torch_ref"]
    owners = timing.KernelOwners(names, op_types={n: cat[n].meta.op_type for n in names})
    table, unowned = timing.kernel_table(str(folder), owners, skip=1)
    assert table["hip_fa_fp32acc"]["dispatches"] == 2
    assert table["hip_fa_fp32acc"]["mean_us"] == pytest.approx(3.0)      # (2 + 4) / 2 us
    assert table["hip_fa_fp16acc"]["mean_us"] == pytest.approx(5.0)
    assert table["torch_ref"] is None
    assert unowned == {prep: (1, pytest.approx(0.3))}
    assert main(["kernels", str(folder), "--backends", ",".join(names), "--skip", "1"]) == 0
    out = capsys.readouterr().out.splitlines()
    assert out[0].split()[:3] == ["Backend", "Dispatches", "Kernel_us"]
    assert out[1].split()[:3] == ["hip_fa_fp32acc", "2", "3.00"]
    assert out[2].split()[:3] == ["hip_fa_fp16acc", "1", "5.00"]
    assert out[3].startswith("torch_ref") and "N/A" in out[3]
    assert out[4].startswith("(unowned)") and prep in out[4]


# --------------------------------------------------------------------------- CLI

def test_cli_names_configurations_by_c_index_or_case_name():
    from fa_amd.harness.__main__ import resolve_cases

    assert resolve_cases("c3") == [CASES[3]]
    assert resolve_cases("c0, B2_S65536_Q12_KV1_D128_stress,c0") == [CASES[0], CASES[4]]
    assert resolve_cases("all") == list(CASES)
    for bad in ("3", "c9", "B9_S1", ""):
        with pytest.raises(SystemExit):
            resolve_cases(bad)


def test_cli_list_and_build(capsys):
    from fa_amd.harness.__main__ import main

    assert main(["list"]) == 0
    out = capsys.readouterr().out
    assert "c3  B2_S131072_Q12_KV1_D128" in out and "backend torch_ref: type=external (reference)" in out
    with patch("fa_amd.build.build") as build:
        assert main(["build", "--backend", "hip_fa_fp32acc"]) == 0
        build.assert_called_once()
    assert "BUILD hip_fa_fp32acc done" in capsys.readouterr().out


def test_visible_pairs_counts_masked_flops():
    from fa_amd.problem.cases import visible_pairs

    def brute(nq, nk, causal):
        if causal == "none":
            return nq * nk
        off = 0 if causal == "top_left" else nk - nq
        return sum(min(nk, max(0, i + off + 1)) for i in range(nq))

    for nq in (1, 2, 5, 300, 1100):
        for nk in (1, 3, 300, 1100):
            for causal in ("none", "top_left", "bottom_right"):
                assert visible_pairs(nq, nk, causal) == brute(nq, nk, causal), (nq, nk, causal)
    n = 131072
    assert visible_pairs(n, n, "top_left") == n * (n + 1) // 2
    assert Case(1, 8, 2, 1).flops == 4 * 2 * 8 * 8 * 128
