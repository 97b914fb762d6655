"""One-pass against key-split forward on problems with few query tiles.

The one-pass forward runs one work item per 256-row query tile, so a problem
with fewer tiles than the GPU has CUs (a short query range or a small batch
against long keys) leaves CUs idle for its whole duration. The key-split
forward (``fa_fwd_split``) cuts every tile's key range into parts, runs each
(tile, part) as its own work item and merges the parts' (O, lse) pairs. For
each shape this prints the library's automatic part count, the device time
per forward of both paths (HIP events around ``--steps`` forwards after
``--warmup``), the achieved QK/PV TFLOP/s (4 B Hq Nq Nk 128 FLOP) and the
largest difference between the two outputs.

Usage: python -m fa_amd.measure.split [--acc fp32|fp16] [--shape B,Hq,Hkv,Nq,Nk ...]
"""

from __future__ import annotations

import argparse
import os
import sys

# (B, Hq, Hkv, Nq, Nk): the headline's head layout with short query ranges
# against long keys, a single query row per head, and c0 (B1 N4096).
SHAPES = [
    (1, 12, 1, 1, 131072),
    (1, 12, 1, 256, 131072),
    (1, 12, 1, 1024, 131072),
    (1, 12, 1, 4096, 131072),
    (2, 12, 1, 2048, 65536),
    (1, 12, 1, 4096, 4096),
]
PEAK_TFLOPS = 2516.6


def parse_shape(text):
    vals = tuple(int(x) for x in text.split(","))
    if len(vals) != 5:
        raise argparse.ArgumentTypeError("shape is B,Hq,Hkv,Nq,Nk")
    return vals


def measure(shape, acc, warmup, steps, seed=0):
    import torch

    from fa_amd import build
    from fa_amd.binding import AttentionConfig, Operator
    from fa_amd.harness import timing

    if not build.LIBRARY.is_file():
        raise FileNotFoundError(f"{build.LIBRARY} is not built (python -m fa_amd.build)")
    b, hq, hkv, nq, nk = shape
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, nq, 128, generator=g, dtype=torch.float16).cuda()
    k = torch.randn(b, hkv, nk, 128, generator=g, dtype=torch.float16).cuda()
    v = torch.randn(b, hkv, nk, 128, generator=g, dtype=torch.float16).cuda()
    one = Operator(build.LIBRARY, AttentionConfig(acc=acc))
    split = Operator(build.LIBRARY, AttentionConfig(acc=acc, splits=0))
    flops = 4.0 * b * hq * nq * nk * 128
    us_one = timing.device_us(lambda: one(q, k, v), iters=steps, warmup=warmup)
    us_split = timing.device_us(lambda: split(q, k, v), iters=steps, warmup=warmup)
    diff = float((one(q, k, v).float() - split(q, k, v).float()).abs().max())
    return {
        "shape": shape, "parts": split.split_count(q.shape, k.shape),
        "one_us": us_one, "split_us": us_split,
        "one_tflops": flops / us_one / 1e6, "split_tflops": flops / us_split / 1e6,
        "max_diff": diff,
    }


def render(rows, acc, command):
    lines = [f"# one-pass vs key-split forward, hip_fa_{acc}acc (automatic part count), one MI355X",
             f"command: {command}",
             f"{'B,Hq,Hkv,Nq,Nk':<22} {'tiles':>5} {'parts':>5} {'one-pass us':>12} {'TFLOP/s':>8} "
             f"{'split us':>10} {'TFLOP/s':>8} {'speedup':>7} {'max|diff|':>10}"]
    for r in rows:
        b, hq, _, nq, _ = r["shape"]
        tiles = b * hq * -(-nq // 256)
        lines.append(f"{','.join(map(str, r['shape'])):<22} {tiles:>5} {r['parts']:>5} "
                     f"{r['one_us']:>12.1f} {r['one_tflops']:>8.1f} {r['split_us']:>10.1f} "
                     f"{r['split_tflops']:>8.1f} {r['one_us'] / r['split_us']:>6.2f}x "
                     f"{r['max_diff']:>10.2e}")
    lines.append(f"(TFLOP/s = 4 B Hq Nq Nk 128 / time; nominal dense FP16 peak {PEAK_TFLOPS})")
    return lines


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--acc", default="fp32", choices=("fp32", "fp16"))
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
    for shape in args.shape or SHAPES:
        print(f"measuring {shape}", flush=True)
        rows.append(measure(shape, args.acc, args.warmup, args.steps))
    lines = render(rows, args.acc, args.command or "python -m fa_amd.measure.split")
    print("\n".join(lines), flush=True)
    if args.out:
        with open(args.out, "w", encoding="utf-8") as f:
            f.write("\n".join(lines) + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
