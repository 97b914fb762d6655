"""The harness end to end on the GPU: catalog -> prepare -> bind -> timed
calls -> check against the reference backend (torch_ref), the command-line
check, and bench.py's JSON line."""

import json
import os
import subprocess
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_report_rows_c0():
    from fa_amd.harness import report
    from fa_amd.harness.catalog import Catalog
    from fa_amd.problem.cases import CASES

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    print("case report c0: torch_ref vs hip_fa_fp32acc, hip_fa_fp16acc", flush=True)
    rows = report.run_case(Catalog.default(), CASES[0], ["hip_fa_fp32acc", "hip_fa_fp16acc"],
                           iters=3)
    by = {r.backend: r for r in rows}
    assert by["torch_ref"].check == "ref"
    for n in ("hip_fa_fp32acc", "hip_fa_fp16acc"):
        row = by[n]
        print(f"  {row.cells()}", flush=True)
        assert row.check == "PASS", row
        assert row.max_diff <= 1e-2 and row.avg_us > 0 and row.tflops > 0


def test_cli_check_subprocess():
    print("case python -m fa_amd.harness check hip_fa_fp32acc c0", flush=True)
    r = subprocess.run([sys.executable, "-m", "fa_amd.harness", "check", "--backend",
                        "hip_fa_fp32acc", "--case", "c0"], cwd=REPO,
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=300)
    print(r.stdout[-500:], flush=True)
    assert r.returncode == 0
    assert "CHECK B1_S4096_Q12_KV1_D128 backend=hip_fa_fp32acc PASS" in r.stdout


@pytest.mark.parametrize("causal", ["none", "top_left"])
def test_bench_json_line(causal):
    """bench.py's one JSON line at c0: the fields the driver reads, the roofline
    consistent with the value, and the CPU baseline of the oracle port on c0."""
    print(f"case bench.py c0 causal={causal}", flush=True)
    proc = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--case", "0",
                           "--steps", "3", "--warmup", "1", "--cpu-seconds", "1",
                           "--causal", causal, "--configs", "0,1"],
                          capture_output=True, text=True, timeout=240)
    assert proc.returncode == 0, proc.stderr[-2000:]
    line = json.loads(proc.stdout.strip().splitlines()[-1])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
                "roofline", "cpu_baseline"):
        assert key in line, key
    assert line["n_gpus"] == 1 and line["steps"] == 3 and line["value"] > 0
    assert line["config"]["causal"] == causal and line["config"]["tile"].startswith("pp_")
    roof = line["roofline"]
    assert roof["bound"] == "mfma" and abs(roof["frac"] - line["value"] / roof["peak"]) < 1e-3
    cpu = line["cpu_baseline"]
    assert cpu["kind"] == "port" and cpu["value"] > 0 and cpu["cores"] == os.cpu_count()
    assert cpu["sample"].startswith("c0 B1_S4096_Q12_KV1_D128: the full forward")
    # Both variants of the configurations asked for, full attention; the
    # headline's own entry is the headline measurement when it is one of them.
    table = line["configs"]
    assert sorted(table) == ["c0", "c1"]
    assert table["c1"]["workload"] == "B1_S32768_Q12_KV1_D128"
    for row in table.values():
        for acc in ("fp32", "fp16"):
            assert row[acc]["ms"] > 0 and row[acc]["tflops"] > 0
    if causal == "none":
        assert table["c0"]["fp32"]["ms"] == round(line["ms_per_step"], 4)
