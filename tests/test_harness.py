"""Host-only regressions for the plugin API, the drivers and the harness.

Mirror the intent of the reference's host tests
(tests/test_external_ascendc.py, tests/test_kernel_names.py): driver selection
and compile policy, the reference backend's exact call, deferred adaptation,
prepare-before-inputs ordering in the bench, compile-phase task selection,
project validation and build/load ordering for the hip driver, and exact
kernel-name attribution in the profiler. Everything runs on the CPU with
mocks and a synthetic project directory.
"""

import subprocess
import sys
import tempfile
import unittest
from pathlib import Path
from types import SimpleNamespace
from unittest.mock import Mock, patch

from fa_amd.core import contract, profiler, registry
from fa_amd.core.drivers import external, hip


class ExternalTests(unittest.TestCase):
    def test_registration_and_precompile_selection(self):
        prebuilt = SimpleNamespace(META=SimpleNamespace(type="external"))
        source = SimpleNamespace(META=prebuilt.META, build=Mock())
        self.assertIs(registry.driver_for(prebuilt.META), external)
        self.assertFalse(registry.needs_compile(prebuilt))
        self.assertTrue(registry.needs_compile(source))
        self.assertTrue(registry.needs_compile(SimpleNamespace(META=SimpleNamespace(type="hip"))))

    def test_unknown_types_are_rejected(self):
        for kind in ("torch", "ascendc", "tilelang"):
            with self.assertRaises(KeyError):
                registry.driver_for(SimpleNamespace(type=kind))

    def test_reference_backend_uses_external_driver_and_exact_formula_call(self):
        from fa_amd.backends.torch_ref import backend

        self.assertEqual(backend.META.type, "external")
        self.assertIs(registry.driver_for(backend.META), external)
        self.assertFalse(registry.needs_compile(backend))
        self.assertTrue(backend.META.is_reference)
        canonical = {name: object() for name in ("q", "k", "v")}
        case = SimpleNamespace(heads_q=12, scale=0.125)
        output = object()
        with patch.object(backend, "attention", Mock(return_value=output)) as attn:
            external.compile(backend, case)
            call = external.make_call(backend, case, canonical)
            attn.assert_not_called()
            self.assertIs(call(), output)
            self.assertIs(call(), output)
        self.assertEqual(attn.call_count, 2)
        attn.assert_called_with(canonical["q"], canonical["k"], canonical["v"], 0.125)

    def test_reference_backend_formula_on_cpu(self):
        import torch

        from fa_amd.backends.torch_ref import backend

        g = torch.Generator().manual_seed(0)
        q = torch.randn(1, 4, 64, 128, generator=g).half()
        k = torch.randn(1, 2, 96, 128, generator=g).half()
        v = torch.randn(1, 2, 96, 128, generator=g).half()
        out = backend.attention(q, k, v, 128 ** -0.5, chunk_elems=96 * 16)
        sd = torch.nn.functional.scaled_dot_product_attention(
            q.float(), k.float().repeat_interleave(2, 1), v.float().repeat_interleave(2, 1)).half()
        self.assertLessEqual(float((out.float() - sd.float()).abs().max()), 2 ** -10)

    def test_optional_build_and_opaque_argument_object(self):
        args = {"q": "tensor", "custom": 123}
        spec = SimpleNamespace(adapt=Mock(return_value=args), call=Mock(return_value="out"))
        external.compile(spec, "case")
        call = external.make_call(spec, "case", "canonical")
        spec.adapt.assert_called_once_with("case", "canonical")
        self.assertEqual(call(), "out")
        self.assertEqual(call(), "out")
        self.assertEqual(spec.call.call_count, 2)
        spec.call.assert_called_with(args)
        spec.build = Mock()
        external.compile(spec, "case")
        external.make_call(spec, "case", "canonical")
        self.assertEqual(spec.build.call_count, 2)

    def test_generic_prepare_defers_adaptation_until_inputs_exist(self):
        spec = SimpleNamespace(META=SimpleNamespace(type="external"),
                               adapt=Mock(return_value="args"), call=Mock(return_value="out"))
        bind = registry.prepare_call(spec, "case")
        spec.adapt.assert_not_called()
        call = bind("canonical")
        spec.adapt.assert_called_once_with("case", "canonical")
        self.assertEqual(call(), "out")

    def test_bench_prepares_backends_before_inputs(self):
        from fa_amd.core import bench
        from fa_amd.problem import canonical

        events = []
        spec = SimpleNamespace(META=SimpleNamespace(type="hip", op_type="Test", is_reference=True))

        def prepare(spec, case):
            events.append("load")

            def bind(inputs):
                events.append("adapt")
                return lambda: None

            return bind

        def inputs(case, seed, device=None):
            events.append("inputs")
            return {}

        with (
            patch.object(registry, "get", return_value=spec),
            patch.object(registry, "prepare_call", side_effect=prepare),
            patch.object(canonical, "build_canonical", side_effect=inputs),
            patch.object(bench.torch.cuda, "synchronize", Mock()),
            patch.object(bench.profiler, "profile_case_us", return_value={"test": 1.0}),
        ):
            rows = bench.process_case(0, backend_names=["test"], ref_name="test", iters=1,
                                      do_check=False, seed=0, atol=0, rtol=0)
        self.assertEqual(events, ["load", "inputs", "adapt"])
        self.assertEqual(rows[0][:4], ["B1_S4096_Q12_KV1_D128", "test", "ref", "1.00"])

    def test_bench_skips_a_backend_whose_load_fails(self):
        from fa_amd.core import bench
        from fa_amd.problem import canonical

        good = SimpleNamespace(META=SimpleNamespace(type="external", is_reference=True))
        bad = SimpleNamespace(META=SimpleNamespace(type="hip", is_reference=False))
        specs = {"good": good, "bad": bad}

        import torch

        def prepare(spec, case):
            if spec is bad:
                raise FileNotFoundError("artifacts missing")
            return lambda inputs: (lambda: torch.zeros(2))

        with (
            patch.object(registry, "get", side_effect=specs.__getitem__),
            patch.object(registry, "prepare_call", side_effect=prepare),
            patch.object(canonical, "build_canonical", return_value={}),
            patch.object(bench.torch.cuda, "synchronize", Mock()),
            patch.object(bench.profiler, "profile_case_us",
                         return_value={"good": 2.0, "bad": None}),
        ):
            rows = bench.process_case(0, backend_names=["good", "bad"], ref_name="good",
                                      iters=1, do_check=True, seed=0, atol=0, rtol=0)
        verdict = {r[1]: r[5] for r in rows}
        self.assertEqual(verdict, {"good": "ref", "bad": "ERR"})

    def test_kernel_name_errors_are_not_swallowed(self):
        from fa_amd.core import bench

        spec = SimpleNamespace(META=SimpleNamespace(type="hip"))
        with (
            patch.object(registry, "get", return_value=spec),
            patch.object(registry, "prepare_call",
                         side_effect=contract.KernelNameError("bad symbol")),
        ):
            with self.assertRaises(contract.KernelNameError):
                bench.process_case(0, backend_names=["x"], ref_name="x", iters=1,
                                   do_check=False, seed=0, atol=0, rtol=0)

    def test_bench_selects_source_external_and_hip_projects(self):
        from fa_amd.core import bench

        specs = {
            name: SimpleNamespace(META=SimpleNamespace(type=kind))
            for name, kind in (("prebuilt", "external"), ("source", "external"),
                               ("project", "hip"), ("torch_op", "external"))
        }
        specs["source"].build = Mock()
        seen = []

        def collect(tasks, worker):
            seen.extend(tasks)
            return []

        with (
            patch.object(registry, "_BACKENDS", specs),
            patch.object(bench.schedule, "parallel_compile", side_effect=collect),
        ):
            bench.compile_phase(list(specs), [0, 1])
        self.assertEqual(seen, [("source", 0), ("source", 1), ("project", 0), ("project", 1)])


class RegistryTests(unittest.TestCase):
    def test_discovery_keys_by_directory_with_one_reference(self):
        names = registry.all_names()
        self.assertEqual(sorted(names), ["hip_fa_fp16acc", "hip_fa_fp32acc", "torch_ref"])
        ref_name, ref = registry.get_reference()
        self.assertEqual(ref_name, "torch_ref")
        for n in names:
            self.assertEqual(registry.name_of(registry.get(n)), n)

    def test_registry_rejects_unregistered_or_ambiguous_module(self):
        spec = SimpleNamespace(META=SimpleNamespace(diagnostic=False))
        for registered in ({}, {"one": spec, "two": spec}):
            with patch.object(registry, "_BACKENDS", registered):
                with self.assertRaises(ValueError):
                    registry.name_of(spec)

    def test_reference_must_be_unique(self):
        ref = SimpleNamespace(META=SimpleNamespace(is_reference=True))
        for registered in ({}, {"a": ref, "b": ref}):
            with patch.object(registry, "_BACKENDS", registered):
                with self.assertRaises(ValueError):
                    registry.get_reference()

    def test_diagnostic_backends_are_not_attention(self):
        diag = SimpleNamespace(META=SimpleNamespace(diagnostic=True))
        with patch.object(registry, "_BACKENDS", {"diag": diag}):
            self.assertEqual(registry.all_names(), [])
            self.assertEqual(registry.all_names(include_diagnostics=True), ["diag"])
            with self.assertRaisesRegex(ValueError, "diagnostic"):
                registry.require_attention(diag)

    def test_hip_backends_declare_kernel_symbols_containing_their_names(self):
        for n in ("hip_fa_fp32acc", "hip_fa_fp16acc"):
            meta = registry.get(n).META
            self.assertEqual(meta.type, "hip")
            self.assertTrue(meta.op_type.startswith(n))


class HipProjectTests(unittest.TestCase):
    def setUp(self):
        self.temp = tempfile.TemporaryDirectory()
        self.addCleanup(self.temp.cleanup)
        self.root = Path(self.temp.name)
        (self.root / "csrc").mkdir()
        (self.root / "csrc" / "op.hip").write_text("// structure fixture, not a kernel\n")

    def spec(self, command=()):
        project = hip.Project(self.root, ("build/libop.so",), command)
        operator = Mock(return_value="canonical output")
        return SimpleNamespace(project=Mock(return_value=project),
                               load=Mock(return_value=operator),
                               adapt=Mock(return_value=("q", "k", "v")))

    def test_generic_backend_is_rejected(self):
        spec = SimpleNamespace(adapt=Mock(), call=Mock())
        with self.assertRaisesRegex(TypeError, 'type="external"'):
            hip.compile(spec, "case")
        spec.adapt.assert_not_called()
        spec.call.assert_not_called()

    def test_prepare_loads_without_adapting_or_launching(self):
        (self.root / "build").mkdir()
        (self.root / "build/libop.so").write_bytes(b"test fixture")
        spec = self.spec()
        spec.META = SimpleNamespace(type="hip")
        bind = registry.prepare_call(spec, "case")
        spec.load.assert_called_once()
        spec.adapt.assert_not_called()
        spec.load.return_value.assert_not_called()
        call = bind("canonical")
        spec.adapt.assert_called_once_with("case", "canonical")
        self.assertEqual(call(), "canonical output")

    def test_structural_validation_precedes_build(self):
        (self.root / "csrc" / "op.hip").unlink()
        with patch.object(hip.subprocess, "run") as run:
            with self.assertRaisesRegex(ValueError, "csrc"):
                hip.compile(self.spec(("unused",)), "case")
            run.assert_not_called()

    def test_explicit_build_outputs_load_and_call(self):
        command = (sys.executable, "-c",
                   "from pathlib import Path; Path('build').mkdir(exist_ok=True); "
                   "Path('build/libop.so').write_bytes(b'host-test artifact, not ELF')")
        spec = self.spec(command)
        hip.compile(spec, "case")
        self.assertTrue((self.root / "build/libop.so").is_file())
        spec.load.assert_not_called()  # the CPU build never loads the library
        call = hip.make_call(spec, "case", "canonical")
        spec.load.assert_called_once_with("case", spec.project.return_value)
        spec.adapt.assert_called_once_with("case", "canonical")
        self.assertEqual(call(), "canonical output")
        spec.load.return_value.assert_called_once_with("q", "k", "v")

    def test_prebuilt_project_requires_declared_outputs(self):
        spec = self.spec()
        with self.assertRaises(FileNotFoundError):
            hip.make_call(spec, "case", "canonical")
        spec.load.assert_not_called()
        (self.root / "build").mkdir()
        (self.root / "build/libop.so").write_bytes(b"fixture")
        with patch.object(hip.subprocess, "run") as run:
            hip.compile(spec, "case")
            run.assert_not_called()

    def test_failed_build_never_loads_or_runs(self):
        spec = self.spec((sys.executable, "-c", "raise SystemExit(3)"))
        with self.assertRaises(subprocess.CalledProcessError):
            hip.make_call(spec, "case", "canonical")
        spec.load.assert_not_called()
        spec.adapt.assert_not_called()

    def test_invalid_recipe_and_escaping_artifacts_rejected(self):
        for project in (hip.Project(self.root, ("../escape.so",)),
                        hip.Project(self.root, ("/absolute.so",)),
                        hip.Project(self.root, ()),
                        hip.Project(self.root, ("build/lib.so",), "bash build.sh"),
                        hip.Project(self.root, ("build/lib.so",), (), 0)):
            with self.subTest(project=project), self.assertRaises((ValueError, TypeError)):
                project.validate()

    def test_binding_and_argument_contracts_checked(self):
        (self.root / "build").mkdir()
        (self.root / "build/libop.so").write_bytes(b"fixture")
        spec = self.spec()
        spec.load.return_value = None
        with self.assertRaisesRegex(TypeError, "callable binding"):
            hip.make_call(spec, "case", "canonical")
        spec.load.return_value = Mock()
        spec.adapt.return_value = {"q": "not a tuple"}
        with self.assertRaisesRegex(TypeError, "positional-argument tuple"):
            hip.make_call(spec, "case", "canonical")

    def test_real_project_recipe_is_valid_and_needs_no_process_when_current(self):
        from fa_amd import build
        from fa_amd.backends import hip_common

        project = hip_common.project(None)
        project.validate()
        if build.up_to_date():
            self.assertEqual(project.build_command, ())


class ProfileNameTests(unittest.TestCase):
    def test_exact_symbols_disambiguate_prefixes(self):
        names = ["hip_fa", "hip_fa_v3", "torch_ref"]
        symbols = {n: f"{n}_kernel" for n in names[:2]}
        op_types = {n: "main_kernel" for n in names[:2]}
        op_types["torch_ref"] = "Cijk"
        expected = {
            "hip_fa_kernel": "hip_fa",
            "hip_fa_v3_kernel": "hip_fa_v3",
            "main_kernel": None,
            "hip_fa_v30_kernel": None,
            "prefix_hip_fa_v3_kernel": None,
            "Cijk_Alik_Bljk_S": "torch_ref",
        }
        for symbol, backend in expected.items():
            with self.subTest(symbol=symbol):
                self.assertEqual(profiler._match_backend(symbol, names, op_types, symbols), backend)

    def test_mangled_hip_kernels_attribute_by_directory_name(self):
        names = ["hip_fa_fp32acc", "hip_fa_fp16acc", "torch_ref"]
        op_types = {n: registry.get(n).META.op_type for n in names}
        k32 = "_ZN12_GLOBAL__N_121hip_fa_fp32acc_kernelILi1ELi2ELi1ELi128ELi2EEEvPKDF16_S2_S2_PDF16_iiiif"
        k16 = k32.replace("fp32acc", "fp16acc")
        self.assertEqual(profiler._match_backend(k32, names, op_types, {}), "hip_fa_fp32acc")
        self.assertEqual(profiler._match_backend(k16, names, op_types, {}), "hip_fa_fp16acc")
        self.assertIsNone(profiler._match_backend("fa_prep_kernel", names, op_types, {}))

    def test_kernel_trace_averages(self):
        with tempfile.NamedTemporaryFile("w", suffix=".csv", delete=False) as f:
            f.write('"Kernel_Name","Start_Timestamp","End_Timestamp"\n')
            f.write('"x_hip_fa_fp32acc_kernel_y",1000,3000\n"x_hip_fa_fp32acc_kernel_y",5000,9000\n')
            f.write('"other",0,100\n')
        got = profiler.kernel_times_us(f.name, ["hip_fa_fp32acc", "torch_ref"])
        Path(f.name).unlink()
        self.assertEqual(got, {"hip_fa_fp32acc": 3.0, "torch_ref": None})


if __name__ == "__main__":
    unittest.main()


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
