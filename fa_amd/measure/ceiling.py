"""The board's sustained dense FP16 matrix rate, the ceiling the attention kernel runs under.

Two measurements, both on the GPU, both timed with HIP events on torch's
current stream after warmup launches:

* ``mfma_loop`` -- ``libfa_ceiling.so``: every SIMD of every CU issuing
  nothing but ``v_mfma_f32_32x32x16_f16`` (the attention kernel's matrix
  instruction) from two waves, in the attention kernel's launch shape, with
  random FP16 operands either in registers (mode 0), with each A operand
  read from LDS first (mode 1), or with that LDS traffic plus the attention
  softmax's VALU instruction mix beside every MFMA (mode 2: one exponential
  and three other FP32 operations, independent of the MFMAs -- the forward's
  work without its dependencies and barriers), or with each LDS read
  feeding two MFMAs (mode 3: half the LDS traffic), or with both operands
  read from LDS (mode 4: twice the traffic, a test of LDS bandwidth), or
  with one wave per SIMD and each LDS read feeding two MFMAs, alone (mode
  5) or with the softmax's VALU mix in the same wave (mode 6): the
  single-wave layout a 64-row-per-wave tile would need. Modes 7-12 run the
  attention kernel's own skeleton -- its registers, its MFMA step and its
  two-group ping-pong with a barrier per phase -- with the softmax's VALU
  step left out (7), whole (9; 8 with the row sum by FP16 dot products, as
  the kernel had it before), or without its exponentials (10), its FP16
  packing and row sum (11) or its row sum (12): what each part of the
  softmax costs beside the matrix products. Its trace records give the clock it ran at.
* ``gemm`` -- torch's FP16 matrix product (hipBLASLt) on large square and
  rectangular shapes, the rate a tuned vendor GEMM reaches.

The MI355X's nominal dense FP16 peak, 2516.6 TFLOP/s, assumes every CU at
2.4 GHz; under sustained matrix load the board lowers its clock to stay within
its power limit, so these rates (and the clock the loop reports) are the
practical ceiling an MFMA-bound kernel is measured against.

``python -m fa_amd.measure.ceiling [--out FILE]`` prints (and writes) the
summary; ``measure()`` returns it as a dict for bench.py.
"""

from __future__ import annotations

import argparse
import ctypes as C
import os
import sys

GEMM_SHAPES = ((8192, 8192, 8192), (8192, 8192, 16384), (16384, 16384, 8192))
# MFMA loop modes of libfa_ceiling.so and their labels in measure()'s result.
MODES = ((0, "registers"), (1, "lds_operand"), (2, "lds_operand_softmax_valu"),
         (3, "lds_operand_read_per_two"), (4, "both_operands_lds"),
         (5, "one_wave_read_per_two"), (6, "one_wave_read_per_two_softmax_valu"),
         (7, "pingpong_no_softmax"), (8, "pingpong_softmax_dot2_rowsum"),
         (9, "pingpong_softmax"), (10, "pingpong_softmax_no_exp"),
         (11, "pingpong_softmax_no_pack_no_rowsum"), (12, "pingpong_softmax_no_rowsum"))
MODE_TITLES = {0: "operands in registers", 1: "A operand read from LDS",
               2: "A operand from LDS + the softmax's VALU mix",
               3: "one LDS operand read per two MFMAs", 4: "both operands read from LDS",
               5: "one wave per SIMD, one LDS read per two MFMAs",
               6: "one wave per SIMD, one LDS read per two MFMAs + the VALU mix in-wave",
               7: "attention skeleton: ping-pong MFMA steps and barriers, no softmax",
               8: "attention skeleton + softmax, row sum by v_dot2c_f32_f16",
               9: "attention skeleton + softmax as the kernel runs it (row sum by v_fma_mix_f32)",
               10: "attention skeleton + softmax without the exponentials",
               11: "attention skeleton + softmax without FP16 packing and row sum",
               12: "attention skeleton + softmax without the row sum"}
# Loop iterations per workgroup: 16 MFMAs per wave and iteration in modes
# 0-6, one 64-MFMA step (two phases) in the ping-pong modes.
ITERS = {m: (2048 if m >= 7 else 16384) for m, _ in MODES}


def _library():
    from fa_amd import build

    lib = C.CDLL(str(build.CEILING.library), mode=C.RTLD_LOCAL)
    lib.fa_ceiling_flops_per_workgroup.restype = C.c_uint64
    lib.fa_ceiling_flops_per_workgroup.argtypes = [C.c_int]
    lib.fa_ceiling_threads.restype = C.c_int
    lib.fa_ceiling_threads.argtypes = [C.c_int]
    lib.fa_ceiling_flops.restype = C.c_uint64
    lib.fa_ceiling_flops.argtypes = [C.c_int, C.c_int]
    lib.fa_ceiling_mfma.restype = C.c_int
    lib.fa_ceiling_mfma.argtypes = [C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                                    C.c_void_p, C.c_void_p]
    return lib


def mfma_loop(mode, workgroups=2048, iters=None, reps=3, warmup=2):
    """(TFLOP/s, trace records) of the MFMA-only kernel in ``mode``."""
    import torch

    if iters is None:
        iters = ITERS[mode]
    lib = _library()
    g = torch.Generator().manual_seed(7)
    operands = torch.randn(8192, generator=g).half().cuda()
    threads = lib.fa_ceiling_threads(mode)
    if threads <= 0:
        raise ValueError(f"unknown MFMA loop mode {mode}")
    out = torch.empty(workgroups * threads, dtype=torch.float32, device="cuda")
    trace = torch.zeros(workgroups, 8, dtype=torch.int64, device="cuda")
    stream = torch.cuda.current_stream()

    def launch(with_trace):
        rc = lib.fa_ceiling_mfma(mode, workgroups, iters, operands.data_ptr(), out.data_ptr(),
                                 trace.data_ptr() if with_trace else None,
                                 C.c_void_p(stream.cuda_stream))
        if rc:
            raise RuntimeError(f"fa_ceiling_mfma failed with status {rc}")

    for _ in range(warmup):
        launch(False)
    torch.cuda.synchronize()
    begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    begin.record(stream)
    for _ in range(reps):
        launch(False)
    end.record(stream)
    torch.cuda.synchronize()
    seconds = begin.elapsed_time(end) / 1e3 / reps
    launch(True)
    torch.cuda.synchronize()
    if not torch.isfinite(out).all():
        raise RuntimeError("MFMA ceiling kernel produced non-finite sums")
    flops = lib.fa_ceiling_flops(mode, iters) * workgroups
    return flops / seconds / 1e12, trace.cpu().numpy()


def gemm(shapes=GEMM_SHAPES, reps=20, warmup=3):
    """{(m, n, k): TFLOP/s} of torch FP16 matmul (A [m,k] @ B [k,n], N(0,1) data)."""
    import torch

    rates = {}
    g = torch.Generator().manual_seed(11)
    for m, n, k in shapes:
        a = torch.randn(m, k, generator=g).half().cuda()
        b = torch.randn(k, n, generator=g).half().cuda()
        for _ in range(warmup):
            a @ b
        torch.cuda.synchronize()
        begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        begin.record()
        for _ in range(reps):
            a @ b
        end.record()
        torch.cuda.synchronize()
        rates[(m, n, k)] = 2.0 * m * n * k * reps / (begin.elapsed_time(end) / 1e3) / 1e12
        del a, b
    return rates


# The loops bench.py measures beside the forward: the MFMA-only loops and
# the attention skeleton with its whole softmax step.
BENCH_MODES = (0, 1, 2, 3, 7, 9)


def measure(gemm_reps=20, modes=BENCH_MODES):
    from fa_amd.measure import clock

    out = {"gemm_tflops": {}, "mfma_loop": {}}
    for shape, rate in gemm(reps=gemm_reps).items():
        out["gemm_tflops"]["x".join(map(str, shape))] = round(rate, 1)
    for mode, label in MODES:
        if mode not in modes:
            continue
        rate, records = mfma_loop(mode)
        s = clock.summarize(records)
        out["mfma_loop"][label] = {"tflops": round(rate, 1),
                                   "clock_mhz": round(s["mean_mhz_time_weighted"], 0)}
    out["gemm_best_tflops"] = max(out["gemm_tflops"].values())
    out["mfma_loop_best_tflops"] = max(v["tflops"] for v in out["mfma_loop"].values())
    out["softmax_mix_loop_tflops"] = out["mfma_loop"]["lds_operand_softmax_valu"]["tflops"]
    if "pingpong_softmax" in out["mfma_loop"]:
        out["skeleton_tflops"] = out["mfma_loop"]["pingpong_softmax"]["tflops"]
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--out")
    ap.add_argument("--command", default="")
    ap.add_argument("--records", help="save the loop's trace records as <prefix>_mode<m>.npy")
    ap.add_argument("--no-gemm", action="store_true",
                    help="run only the MFMA loops (no vendor GEMM before them)")
    ap.add_argument("--modes", help="comma-separated loop modes (default: all)")
    args = ap.parse_args(argv)
    repo = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    if repo not in sys.path:
        sys.path.insert(0, repo)
    from fa_amd.measure import clock

    lines = ["# sustained dense FP16 matrix rate of this board (nominal peak 2516.6 TFLOP/s)",
             f"command: {args.command or 'python -m fa_amd.measure.ceiling ' + ' '.join(argv or sys.argv[1:])}"]
    for shape, rate in ({} if args.no_gemm else gemm()).items():
        lines.append(f"gemm_fp16 {shape[0]}x{shape[1]}x{shape[2]} (torch.matmul, hipBLASLt): "
                     f"{rate:.1f} TFLOP/s = {rate / clock.PEAK_TFLOPS:.3f} of nominal")
        print(lines[-1], flush=True)
    modes = [int(m) for m in args.modes.split(",")] if args.modes else [m for m, _ in MODES]
    for mode in modes:
        label = MODE_TITLES[mode]
        rate, records = mfma_loop(mode)
        if args.records:
            import numpy as np

            np.save(f"{args.records}_mode{mode}.npy", records)
        s = clock.summarize(records)
        f = s["mean_mhz_time_weighted"]
        lines.append(f"mfma_loop mode {mode} ({label}): {rate:.1f} TFLOP/s = "
                     f"{rate / clock.PEAK_TFLOPS:.3f} of nominal; clock {f:.0f} MHz "
                     f"(p10 {s['p10_mhz']:.0f}, p90 {s['p90_mhz']:.0f}); "
                     f"{rate / clock.roof_at(f):.3f} of the roof at that clock")
        print(lines[-1], flush=True)
    if args.out:
        with open(args.out, "w", encoding="utf-8") as fh:
            fh.write("\n".join(lines) + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
