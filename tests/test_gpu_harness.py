"""The reference-style harness end to end on the GPU: registry -> prepare_call
-> bind -> timed calls -> check against the reference backend (torch_ref),
as the reference's ``core/bench.py:80-153`` runs one case."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_bench_process_case_c0():
    from fa_amd.core import bench, registry

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    print("case harness c0: torch_ref vs hip_fa_fp32acc, hip_fa_fp16acc", flush=True)
    names = ["torch_ref", "hip_fa_fp32acc", "hip_fa_fp16acc"]
    for n in names:
        registry.require_attention(registry.get(n))
    rows = bench.process_case(0, backend_names=names, ref_name="torch_ref", iters=3,
                              do_check=True, seed=0, atol=1e-2, rtol=1e-2)
    by_name = {r[1]: r for r in rows}
    assert by_name["torch_ref"][2] == "ref"
    for n in ("hip_fa_fp32acc", "hip_fa_fp16acc"):
        row = by_name[n]
        print(f"  {row}", flush=True)
        assert row[5] == "PASS", row
        assert float(row[6]) <= 1e-2
        assert float(row[3]) > 0 and float(row[7]) > 0        # Avg_us, TFLOPS


def test_runner_check_mode_subprocess():
    import os
    import subprocess
    import sys

    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("case runner --mode check hip_fa_fp32acc c0", flush=True)
    r = subprocess.run([sys.executable, "-m", "fa_amd.core.runner", "--backend", "hip_fa_fp32acc",
                        "--case-index", "0", "--mode", "check"], cwd=repo,
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=300)
    print(r.stdout[-500:], flush=True)
    assert r.returncode == 0
    assert "CHECK B1_S4096_Q12_KV1_D128 backend=hip_fa_fp32acc PASS" in r.stdout


@pytest.mark.parametrize("causal", ["none", "top_left"])
def test_bench_json_line(causal):
    """bench.py's one JSON line at c0: the fields the driver reads, the roofline
    consistent with the value, and the CPU baseline of the oracle port."""
    import json
    import os
    import subprocess
    import sys

    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print(f"case bench.py c0 causal={causal}", flush=True)
    proc = subprocess.run([sys.executable, os.path.join(repo, "bench.py"), "--case", "0",
                           "--steps", "3", "--warmup", "1", "--cpu-seconds", "1",
                           "--causal", causal], capture_output=True, text=True, timeout=240)
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
    assert cpu["kind"] == "port" and cpu["value"] > 0 and cpu["cores"] >= 1
