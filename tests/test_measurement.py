"""Host-side measurement helpers: rocprofv3 summaries and bench.py's traffic lookup."""

import csv
import os
import sqlite3

import pytest

from fa_amd.measure import kernel_stats, traffic

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

HEADER = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id",
          "Grid_Size", "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size",
          "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count", "SGPR_Count", "Counter_Name",
          "Counter_Value", "Start_Timestamp", "End_Timestamp"]


def write_counters(folder, counter, rows):
    os.makedirs(folder, exist_ok=True)
    with open(os.path.join(folder, "run_counter_collection.csv"), "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(HEADER)
        for dispatch, name, value in rows:
            rec = dict.fromkeys(HEADER, "0")
            rec.update(Dispatch_Id=str(dispatch), Kernel_Name=name, Counter_Name=counter,
                       Counter_Value=str(value))
            w.writerow([rec[h] for h in HEADER])


def test_traffic_scales_by_the_calibration_kernel(tmp_path):
    attn, copy = "hip_fa_fp32acc_kernel<1>", "elementwise bitwise_not kernel"
    # Per-dispatch values are summed over rows (channels); the calibration
    # kernel under-reads fetches by 2x, which the factor undoes.
    write_counters(tmp_path / "f", "FETCH_SIZE", [
        (1, attn, 600.0), (1, attn, 400.0), (2, attn, 1000.0), (3, copy, 512.0)])
    write_counters(tmp_path / "w", "WRITE_SIZE", [(1, attn, 10.0), (2, attn, 10.0), (3, copy, 1024.0)])
    s = traffic.summarize(str(tmp_path / "f"), str(tmp_path / "w"), copy_mib=1,
                          attn_needle="hip_fa_", copy_needle="bitwise_not")
    assert s["fetch_kib"] == 1000.0 and s["write_kib"] == 10.0
    assert s["fetch_factor"] == pytest.approx(2.0) and s["write_factor"] == pytest.approx(1.0)
    assert s["fetch_bytes"] == pytest.approx(2000.0 * 1024)
    assert s["write_bytes"] == pytest.approx(10.0 * 1024)


def test_traffic_requires_one_matching_kernel(tmp_path):
    write_counters(tmp_path / "f", "FETCH_SIZE", [(1, "a", 1.0)])
    write_counters(tmp_path / "w", "WRITE_SIZE", [(1, "a", 1.0)])
    with pytest.raises(ValueError):
        traffic.summarize(str(tmp_path / "f"), str(tmp_path / "w"), copy_mib=1)


def test_kernel_stats_from_rocpd_db(tmp_path):
    db = tmp_path / "out" / "run_results.db"
    db.parent.mkdir()
    con = sqlite3.connect(db)
    con.execute("CREATE TABLE kernels (name TEXT, duration INTEGER)")
    con.executemany("INSERT INTO kernels VALUES (?, ?)",
                    [("hip_fa_fp32acc_kernel", 100), ("hip_fa_fp32acc_kernel", 300), ("fa_prep", 10)])
    con.commit()
    con.close()
    stats = kernel_stats.collect(str(tmp_path / "out"))
    assert stats == {"hip_fa_fp32acc_kernel": [100.0, 300.0], "fa_prep": [10.0]}
    text = kernel_stats.render(stats, flops=2e9, match="hip_fa_fp32acc")
    # 2e9 FLOP / 200 ns average = 1e16 FLOP/s = 10000 TFLOP/s
    assert "10000.0 TFLOP/s" in text
    assert text.splitlines()[1].startswith("hip_fa_fp32acc_kernel")


def test_kernel_stats_skips_warmup_dispatches(tmp_path):
    # A CSV kernel trace written out of launch order: the warmup dispatch
    # (earliest start, slowest) is the one --skip 1 drops.
    folder = tmp_path / "csv"
    folder.mkdir()
    with open(folder / "run_kernel_trace.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writerow(["attn", 300, 400])     # timed step 2: 100 ns
        w.writerow(["attn", 0, 180])       # warmup: 180 ns
        w.writerow(["prep", 290, 300])
        w.writerow(["attn", 200, 290])     # timed step 1: 90 ns
    stats = kernel_stats.collect(str(folder))
    assert stats["attn"] == [180.0, 90.0, 100.0]
    kept = kernel_stats.skip_first(stats, 1)
    assert kept["attn"] == [90.0, 100.0]
    assert kept["prep"] == [10.0]          # a single dispatch is kept
    assert kernel_stats.skip_first(stats, 0) == stats
    # The rocpd database is read in start order when it records one.
    db = tmp_path / "db" / "run_results.db"
    db.parent.mkdir()
    con = sqlite3.connect(db)
    con.execute("CREATE TABLE kernels (name TEXT, start INTEGER, duration INTEGER)")
    con.executemany("INSERT INTO kernels VALUES (?, ?, ?)", [("k", 50, 7), ("k", 10, 9)])
    con.commit()
    con.close()
    assert kernel_stats.collect(str(tmp_path / "db")) == {"k": [9.0, 7.0]}


def test_bench_reads_the_committed_traffic_summary():
    import bench

    key = "hip_fa_fp32acc c3 B2_S131072_Q12_KV1_D128 tile=pp_n128_r2"
    path = os.path.join(REPO, "profiles", "hip_fa_fp32acc_c3_traffic.txt")
    if not os.path.exists(path):
        pytest.skip("no traffic summary committed")
    value = bench.traffic_from_profiles(key)
    assert isinstance(value, int) and value > 1_677_721_600   # at least the algorithmic bytes
    assert bench.traffic_from_profiles(key + "x") is None
    # The JSON line says where the number comes from: not the timed run.
    value2, source = bench.traffic_record(key)
    assert value2 == value and source.startswith("profiles/hip_fa_fp32acc_c3_traffic.txt")
    assert "not measured in this run" in source
    assert bench.traffic_record(key + "x") == (None, None)


def test_counter_summary(tmp_path):
    from fa_amd.measure import counters

    write_counters(tmp_path / "c", "SQ_BUSY_CYCLES", [(1, "hip_fa_fp32acc_kernel", 5.0),
                                                      (1, "hip_fa_fp32acc_kernel", 7.0),
                                                      (2, "hip_fa_fp32acc_kernel", 10.0),
                                                      (3, "fa_prep_kernel", 1.0)])
    assert counters.counter_names(str(tmp_path / "c")) == ["SQ_BUSY_CYCLES"]
    s = counters.summarize(str(tmp_path / "c"), "hip_fa_", ["SQ_BUSY_CYCLES"])
    val, n, kernel = s["SQ_BUSY_CYCLES"]
    assert (n, kernel) == (2, "hip_fa_fp32acc_kernel") and val == 11.0   # median of 12, 10


def test_bench_cli_contract():
    import bench

    args = bench.parse_args([])
    assert (args.gpus, args.case, args.causal, args.kernel) == (1, 3, "none", 0)
    assert bench.parse_args(["--causal", "bottom_right"]).causal == "bottom_right"
    assert bench.parse_args([]).configs == "0,1,2,3,4"
    # More than one GPU is refused before anything touches a device.
    assert bench.main(["--gpus", "2"]) == 2


def test_clock_summary_from_trace_records():
    import numpy as np

    from fa_amd.measure import clock

    # Two records on die 1 at 1500 MHz, one on die 3 at 2000 MHz, one empty record.
    rec = np.zeros((4, 8), dtype=np.int64)
    rec[0] = [(1 << 32) | 5, 1000, 2000, 10, 10 + 15_000, 0, 8, 128]     # 1000 ticks = 10 us
    rec[1] = [(1 << 32) | 6, 1000, 3000, 50, 50 + 30_000, 1, 8, 128]
    rec[2] = [(3 << 32) | 7, 500, 1500, 0, 20_000, 2, 8, 128]
    rec[3] = [0, 7, 7, 0, 0, 3, 0, 128]
    assert np.allclose(clock.clocks_mhz(rec), [1500, 1500, 2000])
    s = clock.summarize(rec)
    assert s["records"] == 4 and s["median_mhz"] == 1500
    assert s["per_xcc_median_mhz"] == {1: 1500.0, 3: 2000.0}
    # Weighted by each record's span: (1500*1000 + 1500*2000 + 2000*1000) / 4000.
    assert s["mean_mhz_time_weighted"] == pytest.approx(1625.0)
    assert s["span_ms"] == pytest.approx((3000 - 7) / 1e5)        # first entry: the empty record
    assert clock.roof_at(1200.0) == pytest.approx(2516.6 / 2)
    lines = clock.render("# t", s, achieved_tflops=1000.0)
    assert any(line.startswith("achieved_tflops: 1000.0") for line in lines)
    with pytest.raises(ValueError):
        clock.summarize(rec[3:])


def test_algorithmic_bytes_of_every_configuration():
    from fa_amd.problem.cases import CASES

    # Q + K + V + O, FP16: c3 is 2*12*131072*128*2 (Q) twice plus 2*1*131072*128*2 (K) twice.
    assert traffic.algorithmic_bytes(CASES[3]) == 1_744_830_464
    assert traffic.algorithmic_bytes(CASES[0]) == 2 * (12 + 1) * 4096 * 256
    for case in CASES:
        assert traffic.algorithmic_bytes(case) == 2 * case.batch * (case.heads_q + case.heads_kv) \
            * case.seq_len * case.dim * 2


def test_split_table_render():
    from fa_amd.measure import split

    assert split.parse_shape("1,12,1,256,131072") == (1, 12, 1, 256, 131072)
    with pytest.raises(Exception):
        split.parse_shape("1,12,1")
    rows = [{"shape": (1, 12, 1, 256, 131072), "parts": 21, "tile": "pp_n128_r2", "one_us": 2149.0,
             "split_us": 224.0, "one_tflops": 95.9, "split_tflops": 920.3, "max_diff": 1.2e-4},
            {"shape": (1, 12, 1, 1, 131072), "parts": 256, "tile": "pp_n128_r2_vnat", "one_us": 1511.0,
             "split_us": 27.7, "one_tflops": 0.5, "split_tflops": 29.1, "max_diff": 7.6e-6}]
    lines = split.render(rows, "fp32", "python -m fa_amd.measure.split")
    assert lines[1] == "command: python -m fa_amd.measure.split"
    row = lines[3].split()
    assert row[:4] == ["1,12,1,256,131072", "pp_n128_r2", "12", "21"] and row[8] == "9.59x"
    row = lines[4].split()      # decode: one packed tile
    assert row[:4] == ["1,12,1,1,131072", "pp_n128_r2_vnat", "1", "256"] and row[8] == "54.55x"


def test_split_sweep_render():
    from fa_amd.measure import split

    rows = [((1, 12, 1, 1024, 131072), 16, [(1, 2195.0), (5, 755.0), (16, 760.0)])]
    lines = split.render_sweep(rows, "fp32", "python -m fa_amd.measure.split --sweep")
    assert lines[3] == ("1,12,1,1024,131072: automatic 16 (760 us), fastest 5 (755 us, "
                        "automatic at 1.007x)")
    assert lines[4] == "  1:2195 5:755 16:760"


def test_ceiling_library_host_side():
    """The MFMA ceiling library's launch shapes and FLOP counts, and its
    host-side rejections (no GPU: nothing is launched)."""
    import ctypes as C

    from fa_amd import build
    from fa_amd.measure import ceiling

    if not build.CEILING.library.exists():
        pytest.skip("libfa_ceiling.so is not built")
    lib = ceiling._library()
    per_mfma = 32 * 32 * 16 * 2
    for mode, _ in ceiling.MODES:
        threads = 256 if mode in (5, 6) else 512
        mfmas = 64 if mode >= 7 else 16     # per wave and iteration
        assert lib.fa_ceiling_threads(mode) == threads
        assert lib.fa_ceiling_flops(mode, 5) == threads // 64 * 5 * mfmas * per_mfma
        assert mode in ceiling.MODE_TITLES and ceiling.ITERS[mode] > 0
    assert [m for m, _ in ceiling.MODES] == list(range(13))
    assert set(ceiling.BENCH_MODES) <= {m for m, _ in ceiling.MODES}
    assert lib.fa_ceiling_threads(13) == 0 and lib.fa_ceiling_threads(-1) == 0
    assert lib.fa_ceiling_flops(13, 5) == 0
    assert lib.fa_ceiling_flops_per_workgroup(5) == lib.fa_ceiling_flops(0, 5)
    for bad in ((13, 1, 1, 16, 16), (-1, 1, 1, 16, 16), (0, 0, 1, 16, 16), (0, 1, 0, 16, 16),
                (0, 1, 1, 24, 16), (0, 1, 1, 16, 8)):
        mode, wg, iters, ops, out = bad
        assert lib.fa_ceiling_mfma(mode, wg, iters, C.c_void_p(ops), C.c_void_p(out), None,
                                   None) == 1
