"""Single-shape benchmark of one kernel (--kernel v0|v1|v2).

Counterpart of the reference's bench/single_shape.py:30-99, same options and
output fields: a spot check of the first two requests against an fp32 torch
reference, then the median of 50 HIP-event-timed calls after 10 warmup calls,
KV bytes, speed of light at 8 TB/s and % of it, and the GPU clocks; the result
is also written as JSON under --out-dir. --num-splits 0 selects the split
heuristic. --profile-mode runs the kernel once with no warmup, check or timing
(the reference's --ncu-mode), for `rocprofv3 --pmc` passes.
"""

import argparse
import json
import math
import os
import sys
import time

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, _HERE)
sys.path.insert(0, os.path.join(os.path.dirname(_HERE), "python"))

import cases  # noqa: E402
from binding import KERNELS  # noqa: E402


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--B", type=int, default=32)
    ap.add_argument("--S", type=int, default=8192)
    ap.add_argument("--Hq", type=int, default=32)
    ap.add_argument("--Hkv", type=int, default=8)
    ap.add_argument("--bs", type=int, default=16)
    ap.add_argument("--kernel", choices=sorted(KERNELS), default="v0")
    ap.add_argument("--num-splits", type=int, default=8,
                    help="split-KV segment count (v2 only; 0 = heuristic)")
    ap.add_argument("--profile-mode", action="store_true",
                    help="run the kernel exactly once, no warmup, no timing")
    ap.add_argument("--out-dir", default=os.path.join(_HERE, "results"))
    args = ap.parse_args(argv)

    scale = 1.0 / math.sqrt(cases.D)
    if args.kernel == "v2":
        fn = lambda *a: KERNELS["v2"](*a, num_splits=args.num_splits)  # noqa: E731
    else:
        fn = KERNELS[args.kernel]
    case = cases.make_case([args.S] * args.B, args.Hq, args.Hkv, args.bs, seed=0, qkv_std=0.5)

    if args.profile_mode:
        fn(*case, scale)
        torch.cuda.synchronize()
        return

    max_abs = cases.spot_check(fn, case, scale)
    print(f"spot check on first {min(2, args.B)} requests passed (max-abs={max_abs:.4e})")
    median_ms = cases.time_op(lambda: fn(*case, scale), warmup=10, runs=50)
    kvb = cases.kv_bytes([args.S] * args.B, args.Hkv)
    sol_ms = cases.sol_us(kvb) / 1e3
    pct = sol_ms / median_ms * 100.0
    clocks = cases.gpu_clocks()
    print(f"median_ms   = {median_ms:.4f}")
    print(f"kv_bytes    = {kvb}")
    print(f"sol_ms      = {sol_ms:.4f}")
    print(f"pct_of_sol  = {pct:.2f}%")
    print(f"clocks      = {clocks}")

    result = {
        "kernel": args.kernel, "B": args.B, "S": args.S, "Hq": args.Hq, "Hkv": args.Hkv,
        "bs": args.bs, "num_splits": args.num_splits if args.kernel == "v2" else None,
        "median_ms": median_ms, "kv_bytes": kvb, "sol_ms": sol_ms, "pct_of_sol": pct,
        "clocks": clocks,
    }
    os.makedirs(args.out_dir, exist_ok=True)
    path = os.path.join(args.out_dir, f"{args.kernel}_{args.B}x{args.S}x{args.Hq}x{args.Hkv}"
                        f"x{args.bs}_{time.strftime('%Y%m%d_%H%M%S')}.json")
    with open(path, "w") as f:
        json.dump(result, f, indent=2)
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
