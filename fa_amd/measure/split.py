"""One-pass against key-split forward on problems with few query tiles.

The one-pass forward runs one work item per 256-row query tile, so a problem
with fewer tiles than the GPU has CUs (a short query range or a small batch
against long keys) leaves CUs idle for its whole duration. The key-split
forward (``fa_fwd_split``) cuts every tile's key range into parts, runs each
(tile, part) as its own work item and merges the parts' (O, lse) pairs. For
each shape this prints the library's automatic tile and part count, the device time
per forward of both paths (HIP events around ``--steps`` forwards after
``--warmup``), the achieved QK/PV TFLOP/s (4 B Hq Nq Nk 128 FLOP) and the
largest difference between the two outputs. With ``--sweep`` it times the
split forward at every explicit part count of SWEEP_COUNTS instead, to check
the automatic choice against the fastest count.

Usage: python -m fa_amd.measure.split [--acc fp32|fp16] [--sweep] [--shape B,Hq,Hkv,Nq,Nk ...]
"""

from __future__ import annotations

import argparse
import os
import sys

# (B, Hq, Hkv, Nq, Nk): the headline's head layout with short query ranges
# against long keys, one or a few query rows per head (decode: the group's
# heads share one packed tile), a batched decode with 8 KV heads of 8 query
# heads each, and c0 (B1 N4096). Up to 128 query rows per head (1536 per KV
# head) the automatic tile reads V in its natural layout.
SHAPES = [
    (1, 12, 1, 1, 131072),
    (1, 12, 1, 16, 131072),
    (8, 64, 8, 1, 8192),
    (1, 12, 1, 128, 131072),
    (1, 12, 1, 256, 131072),
    (1, 12, 1, 1024, 131072),
    (1, 12, 1, 4096, 131072),
    (2, 12, 1, 2048, 65536),
    (1, 12, 1, 4096, 4096),
]
PEAK_TFLOPS = 2516.6
# Explicit part counts of the sweep (counts above a shape's key blocks are skipped).
SWEEP_COUNTS = [1, 2, 3, 4, 5, 6, 8, 10, 12, 16, 21, 24, 32, 42, 64, 96, 128, 192, 256]
SWEEP_SHAPES = SHAPES + [(1, 12, 1, 8192, 8192), (1, 12, 1, 2048, 32768), (1, 4, 1, 2048, 131072),
                         (1, 12, 1, 1, 32768)]


def parse_shape(text):
    vals = tuple(int(x) for x in text.split(","))
    if len(vals) != 5:
        raise argparse.ArgumentTypeError("shape is B,Hq,Hkv,Nq,Nk")
    return vals


def _inputs(shape, seed):
    import torch

    from fa_amd import build

    if not build.LIBRARY.is_file():
        raise FileNotFoundError(f"{build.LIBRARY} is not built (python -m fa_amd.build)")
    b, hq, hkv, nq, nk = shape
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(b, h, n, 128, generator=g, dtype=torch.float16).cuda()
                 for h, n in ((hq, nq), (hkv, nk), (hkv, nk)))


def measure(shape, acc, warmup, steps, seed=0):
    from fa_amd import build
    from fa_amd.binding import AttentionConfig, Operator
    from fa_amd.harness import timing

    b, hq, hkv, nq, nk = shape
    q, k, v = _inputs(shape, seed)
    one = Operator(build.LIBRARY, AttentionConfig(acc=acc))
    split = Operator(build.LIBRARY, AttentionConfig(acc=acc, splits=0))
    flops = 4.0 * b * hq * nq * nk * 128
    us_one = timing.device_us(lambda: one(q, k, v), iters=steps, warmup=warmup)
    us_split = timing.device_us(lambda: split(q, k, v), iters=steps, warmup=warmup)
    diff = float((one(q, k, v).float() - split(q, k, v).float()).abs().max())
    return {
        "shape": shape, "parts": split.split_count(q.shape, k.shape),
        "tile": split.kernel_name(q.shape, k.shape),
        "one_us": us_one, "split_us": us_split,
        "one_tflops": flops / us_one / 1e6, "split_tflops": flops / us_split / 1e6,
        "max_diff": diff,
    }


def sweep(shape, acc, warmup, steps, seed=0):
    """(automatic count, [(count, device us)]) over SWEEP_COUNTS and the
    automatic count."""
    from fa_amd import build
    from fa_amd.binding import AttentionConfig, Operator
    from fa_amd.harness import timing

    q, k, v = _inputs(shape, seed)
    auto = Operator(build.LIBRARY, AttentionConfig(acc=acc, splits=0)).split_count(q.shape, k.shape)
    res = []
    for n in sorted(set(SWEEP_COUNTS) | {auto}):
        if n > -(-shape[4] // 128):
            continue
        op = Operator(build.LIBRARY, AttentionConfig(acc=acc, splits=n))
        res.append((n, timing.device_us(lambda: op(q, k, v), iters=steps, warmup=warmup)))
    return auto, res


def render_sweep(rows, acc, command):
    lines = [f"# key-split forward, hip_fa_{acc}acc: device us per forward at each explicit part count,",
             "# against the library's automatic count (one MI355X)",
             f"command: {command}"]
    for shape, auto, res in rows:
        times = dict(res)
        best = min(res, key=lambda r: r[1])
        lines.append(f"{','.join(map(str, shape))}: automatic {auto} ({times[auto]:.0f} us), fastest "
                     f"{best[0]} ({best[1]:.0f} us, automatic at {times[auto] / best[1]:.3f}x)")
        lines.append("  " + " ".join(f"{n}:{us:.0f}" for n, us in res))
    return lines


def render(rows, acc, command):
    lines = [f"# one-pass vs key-split forward, hip_fa_{acc}acc (automatic tile and part count), one MI355X",
             f"command: {command}",
             f"{'B,Hq,Hkv,Nq,Nk':<22} {'tile':<16} {'tiles':>5} {'parts':>5} {'one-pass us':>12} {'TFLOP/s':>8} "
             f"{'split us':>10} {'TFLOP/s':>8} {'speedup':>7} {'max|diff|':>10}"]
    from fa_amd import binding

    for r in rows:
        b, hq, hkv, nq, _ = r["shape"]
        tiles = binding.query_tiles(b, hq, hkv, nq)
        lines.append(f"{','.join(map(str, r['shape'])):<22} {r['tile']:<16} {tiles:>5} {r['parts']:>5} "
                     f"{r['one_us']:>12.1f} {r['one_tflops']:>8.1f} {r['split_us']:>10.1f} "
                     f"{r['split_tflops']:>8.1f} {r['one_us'] / r['split_us']:>6.2f}x "
                     f"{r['max_diff']:>10.2e}")
    lines.append(f"(TFLOP/s = 4 B Hq Nq Nk 128 / time; nominal dense FP16 peak {PEAK_TFLOPS})")
    return lines


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--acc", default="fp32", choices=("fp32", "fp16"))
    ap.add_argument("--sweep", action="store_true", help="time every count of SWEEP_COUNTS")
    ap.add_argument("--shape", type=parse_shape, action="append",
                    help="B,Hq,Hkv,Nq,Nk (repeatable; default: the built-in list)")
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--out", help="also write the table to this file")
    ap.add_argument("--command", default="", help="command line recorded in the table")
    args = ap.parse_args(argv)
    repo = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    if repo not in sys.path:
        sys.path.insert(0, repo)
    rows = []
    command = args.command or "python -m fa_amd.measure.split" + (" --sweep" if args.sweep else "")
    for shape in args.shape or (SWEEP_SHAPES if args.sweep else SHAPES):
        print(f"measuring {shape}", flush=True)
        if args.sweep:
            rows.append((shape,) + sweep(shape, args.acc, args.warmup, args.steps))
        else:
            rows.append(measure(shape, args.acc, args.warmup, args.steps))
    lines = (render_sweep if args.sweep else render)(rows, args.acc, command)
    print("\n".join(lines), flush=True)
    if args.out:
        with open(args.out, "w", encoding="utf-8") as f:
            f.write("\n".join(lines) + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
