"""Benchmark of the gfx950 GQA paged-decode hot path (one decode step).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2]
                    [--kernel v2] [--num-splits 0] [--sweep] [--no-cpu-baseline]

A step is one decode-attention call over the config's whole batch, with every
input resident in HBM. The default workload is BASELINE.json config 2 (32Q/8KV,
d=128, S=8192, B=32, block=16: 1 GiB of K+V), the shape the headline metric is
quoted on; the other configs are selectable with --config.

Timed region: --ramp-seconds of untimed steps (steady clocks), W untimed
steps, then K steps bracketed by
torch.cuda.synchronize(). A v2 step is the C ABI's partial launch followed by
its merge launch (one launch when num_splits is 1) on the current stream, with
a caller-owned workspace. With --num-splits 0 (the default) the step is what
the torch op's automatic choice runs: the token-balanced scan and its merge
where gqa_decode_prefer_balanced says so (configs 4 and 5), else the split
heuristic's count (1 for config 2, 4 for config 3). HIP events are recorded only between groups of steps
(an event between two kernels delays the second):
  value (median us)        median over the groups of the per-step average
  ms_per_step              host wall time of the K steps / K
  roofline.achieved        algorithmic KV bytes / the dominant (partial)
                           kernel's average duration over K back-to-back
                           launches, events around the whole run
The torch operator (what Python callers use, allocation included) is timed
too, the reference's way (bench/common.py:49-64: events around each call,
synchronize after each), as `op_median_us`.

The CPU baseline is the C oracle (oracle/gqa_decode_oracle.c) timed on a
bounded sample of the same workload on this host's cores; its output on the
sample is also compared with the GPU output (spot check, atol=rtol=1e-2).
One JSON line is printed on stdout; progress goes to stderr.
"""

import argparse
import json
import math
import os
import sys
import time

REPO_ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(REPO_ROOT, "mla-decode-kernels_amd")
sys.path.insert(0, os.path.join(PKG_DIR, "python"))
sys.path.insert(0, os.path.join(PKG_DIR, "bench"))

METRIC = ("median µs and % of HBM KV-bytes SoL, 32Q/8KV d=128 S=8192 B=32 block=16")
TRAFFIC_FILE = os.path.join(REPO_ROOT, "profiles", "traffic.txt")


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5"])
    ap.add_argument("--kernel", default="v2", choices=["v0", "v1", "v2", "balanced"],
                    help="v2 with --num-splits 0 makes the op's automatic choice (balanced or split)")
    ap.add_argument("--num-splits", type=int, default=0, help="v2 split count (0 = heuristic)")
    ap.add_argument("--sweep", action="store_true", help="also time v2 over a num_splits sweep")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="oracle threads (default: min(16, cpu count))")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--ramp-seconds", type=float, default=0.5,
                    help="untimed steps before the warmup steps, to reach steady clocks")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="instead: time a plain device copy of MIB MiB (torch.neg into a second "
                         "buffer), the known-size kernel that calibrates rocprofv3's "
                         "FETCH_SIZE / WRITE_SIZE")
    return ap.parse_args(argv)


def read_traffic(config, kernel, num_splits):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3
    counter summary (lines 'config kernel num_splits fetch_bytes write_bytes')."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    with open(TRAFFIC_FILE) as f:
        for line in f:
            parts = line.split()
            if len(parts) == 5 and not line.startswith("#") and parts[:3] == [
                    config, kernel, str(num_splits)]:
                return int(parts[3]) + int(parts[4])
    return None


def kernel_name(kernel, group, balanced=False, hkv=8):
    """The dominant kernel of one step: v0's kernel, else the token-balanced or
    split-rule scan the dispatcher picks: split launches use the matrix cores
    from 5 q-heads per group, the balanced launcher whenever there are 4 or 8
    kv-heads."""
    if kernel == "v0":
        return "gqa_decode_v0_kernel"
    if balanced:
        return ("gqa_decode_balanced_mfma_kernel" if hkv in (4, 8)
                else "gqa_decode_balanced_kernel")
    return "gqa_decode_mfma_kernel" if group >= 5 else "gqa_decode_scan_kernel"


def main(argv=None):
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build measures the decode "
              "path on one GPU (one GPU's share of the batch); run with --gpus 1.",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import capi
    import cases
    from binding import KERNELS, gqa_decode_balanced, gqa_decode_v2

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    props = torch.cuda.get_device_properties(dev)
    if args.copy_probe:
        n = args.copy_probe << 20
        x = torch.ones(n // 4, dtype=torch.float32, device=dev)
        y = torch.empty_like(x)
        ms = cases.time_op(lambda: torch.neg(x, out=y), warmup=3, runs=10)
        print(json.dumps({"copy_probe": "torch.neg fp32", "read_bytes": n, "write_bytes": n,
                          "median_us": round(ms * 1e3, 2),
                          "gbps_read_plus_write": round(2 * n / ms / 1e6, 1)}), flush=True)
        return 0
    cfg = cases.CONFIGS[args.config]
    S_list = cases.config_seq_lens(args.config, args.seed)
    kvb = cases.kv_bytes(S_list, cfg["Hkv"])
    sol = cases.sol_us(kvb)
    scale = 1.0 / math.sqrt(cases.D)
    log(f"config {args.config}: {cfg['desc']}; KV bytes {kvb}; SoL {sol:.2f} us at 8 TB/s")

    t0 = time.time()
    case = cases.make_config_case(args.config, seed=args.seed, device=dev)
    torch.cuda.synchronize()
    log(f"inputs resident in HBM ({time.time() - t0:.1f}s)")
    q, k, v, bt, sl = case
    B, Hq = q.shape[:2]
    Hkv, bs, mb = k.shape[2], k.shape[1], bt.shape[1]

    ns = args.num_splits
    cus = props.multi_processor_count
    # v2 with num_splits 0 makes the torch op's automatic choice: the
    # token-balanced launch where gqa_decode_prefer_balanced says so, else the
    # split heuristic's count.
    balanced = args.kernel == "balanced" or (
        args.kernel == "v2" and ns == 0 and capi.prefer_balanced(B, Hq, Hkv, bs, mb, cus) == 1)
    if args.kernel == "v2" and ns == 0 and not balanced:
        ns = capi.pick_num_splits(B, Hq, Hkv, bs, mb, cus)
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    bal_bytes = capi.balanced_workspace_bytes(B, Hq, Hkv, cus) if balanced else 0
    bal_ws = torch.empty(max(bal_bytes, 4) // 4, dtype=torch.float32, device=dev)

    out = torch.empty_like(q)
    states = B * Hq * max(ns, 1)
    ws = torch.empty(states * (cases.D + 2), dtype=torch.float32, device=dev)
    ws_acc, ws_m, ws_l = ws.data_ptr(), ws.data_ptr() + states * cases.D * 4, \
        ws.data_ptr() + states * (cases.D + 1) * 4
    ptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr())

    def step_parts():
        """One step as its kernel launches through the C ABI."""
        if balanced:
            bal = (*ptrs, out.data_ptr(), B, Hq, Hkv, bs, mb, scale, cus, bal_ws.data_ptr(),
                   bal_bytes, sp)
            return [lambda: capi.balanced_partial_launch(*bal),
                    lambda: capi.balanced_merge_launch(*bal)]
        if args.kernel == "v2" and ns == 1:
            # One split: the single-pass kernel writes out (and the workspace).
            return [lambda: capi.v2_launch(*ptrs, out.data_ptr(), B, Hq, Hkv, bs, mb, scale, 1,
                                           ws_acc, ws_m, ws_l, sp)]
        if args.kernel == "v2":
            return [lambda: capi.v2_partial_launch(*ptrs, B, Hq, Hkv, bs, mb, scale, ns, ws_acc,
                                                   ws_m, ws_l, sp),
                    lambda: capi.v2_merge_launch(ws_acc, ws_m, ws_l, out.data_ptr(), B, Hq, ns,
                                                 sp)]
        launch = capi.v1_launch if args.kernel == "v1" else capi.v0_launch
        return [lambda: launch(*ptrs, out.data_ptr(), B, Hq, Hkv, bs, mb, scale, sp)]

    parts = step_parts()

    def step():
        for p in parts:
            rc = p()
            if rc != 0:
                raise RuntimeError(f"launch failed: hipError_t {rc}")

    # Clock ramp: the GPU takes a few hundred milliseconds of load to reach its
    # steady clocks, far longer than W short steps; run untimed steps for
    # --ramp-seconds first, then the W warmup steps.
    t_ramp = time.perf_counter() + args.ramp_seconds
    while time.perf_counter() < t_ramp:
        for _ in range(8):
            step()
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # Timed region: exactly K steps back to back. Events sit only between
    # groups of steps (an event between two kernels delays the second one), so
    # each group's average is the steady-state step time; value = their median.
    K = args.steps
    groups = max(1, min(10, K // 5))
    bounds = [round(g * K / groups) for g in range(groups + 1)]
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(groups + 1)]
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    for g in range(groups):
        ev[g].record(stream)
        for _ in range(bounds[g + 1] - bounds[g]):
            step()
    ev[groups].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    group_us = sorted(ev[g].elapsed_time(ev[g + 1]) * 1e3 / (bounds[g + 1] - bounds[g])
                      for g in range(groups))
    median_us = group_us[groups // 2]

    # The dominant kernel alone, K launches back to back on the same stream:
    # its average launch duration for the roofline.
    kev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    kev[0].record(stream)
    for _ in range(K):
        if parts[0]() != 0:
            raise RuntimeError("launch failed")
    kev[1].record(stream)
    torch.cuda.synchronize()
    kern_avg_us = kev[0].elapsed_time(kev[1]) * 1e3 / K
    log(f"{args.kernel}: median step {median_us:.2f} us (groups {group_us[0]:.1f}..{group_us[-1]:.1f}), "
        f"dominant kernel avg {kern_avg_us:.2f} us ({kvb / kern_avg_us / 1e3:.1f} GB/s), "
        f"wall {wall / K * 1e3:.3f} ms/step")

    # The torch operator, timed the reference's way.
    if args.kernel == "balanced":
        op = lambda: gqa_decode_balanced(*case, scale)  # noqa: E731
    elif args.kernel == "v2":
        op = lambda: gqa_decode_v2(*case, scale, num_splits=args.num_splits if balanced else ns)  # noqa: E731
    else:
        op = lambda: KERNELS[args.kernel](*case, scale)  # noqa: E731
    op_ms = cases.time_op(op, warmup=3, runs=min(K, 30))
    out_op = op()
    torch.cuda.synchronize()
    assert torch.equal(out_op, out), "torch op and C ABI outputs differ"

    sweep = None
    if args.sweep and args.kernel == "v2":
        sweep = {}
        for s in [1, 2, 4, 8, 16, 32, 64, 128]:
            ms = cases.time_op(lambda: gqa_decode_v2(*case, scale, num_splits=s), 3, 20)
            sweep[s] = round(ms * 1e3, 2)
            log(f"  sweep num_splits={s}: {ms * 1e3:.2f} us ({sol / (ms * 1e3) * 100:.1f}% SoL)")

    split_label = "balanced" if balanced else ns
    traffic = read_traffic(args.config, "v2" if balanced else args.kernel, split_label)
    achieved = kvb / (kern_avg_us * 1e-6) / 1e9
    result = {
        "metric": METRIC,
        "value": round(median_us, 3),
        "unit": "us",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(wall / K * 1e3, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "accum": "fp32",
        "data": f"synthetic N(0,1) bf16, seed {args.seed}",
        "config": {"workload": f"{args.config}: {cfg['desc']}", "Hq": Hq, "Hkv": Hkv, "B": B,
                   "S": cfg["S"] if cfg["S"] else "U[1,32768]", "block": bs,
                   "kernel": args.kernel,
                   "num_splits": split_label if args.kernel in ("v2", "balanced") else None},
        "pct_of_sol": round(sol / median_us * 100, 2),
        "achieved_gbps": round(kvb / median_us / 1e3, 1),
        "kv_bytes": kvb,
        "sol_us": round(sol, 3),
        "op_median_us": round(op_ms * 1e3, 3),
        "roofline": {"bound": "hbm", "kernel": kernel_name(args.kernel, Hq // Hkv, balanced, Hkv),
                     "achieved": round(achieved, 1),
                     "peak": 8000.0, "unit": "GB/s", "frac": round(achieved / 8000.0, 4),
                     "avg_kernel_us": round(kern_avg_us, 3),
                     "traffic": traffic},
        "device": props.name, "gcn_arch": props.gcnArchName, "cus": props.multi_processor_count,
        "clocks": cases.gpu_clocks(),
    }
    if sweep:
        result["sweep_us"] = sweep

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args, case, out, S_list, scale, median_us)
    print(json.dumps(result), flush=True)
    return 0


def cpu_baseline(args, case, out, S_list, scale, gpu_us):
    """The oracle on this host's cores over a bounded sample of the workload
    (whole requests, at most ~10 s per run), scaled to one full step."""
    import numpy as np

    from cases import host_case
    sys.path.insert(0, REPO_ROOT)
    from oracle import c_oracle  # noqa: E402  (the checker, timed as the CPU baseline)

    threads = args.cpu_threads or min(16, os.cpu_count() or 1)
    B = len(S_list)
    # Grow the sample one request at a time until it holds ~1/8 of the step or
    # the estimated run time passes ~10 s; first time one request to calibrate.
    probe = [0]
    hc = host_case(case, probe)
    t0 = time.perf_counter()
    c_oracle.attention_ref(*hc, scale, nthreads=threads)
    per_token = (time.perf_counter() - t0) / max(S_list[0], 1)
    budget_s, sample, tokens = 10.0, [], 0
    for b in range(B):
        if sample and (tokens + S_list[b]) * per_token > budget_s:
            break
        sample.append(b)
        tokens += S_list[b]
    hc = host_case(case, sample)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        ref_out = c_oracle.attention_ref(*hc, scale, nthreads=threads)
        times.append(time.perf_counter() - t0)
    t = sorted(times)[1]
    frac = tokens / sum(S_list)
    cpu_us = t / frac * 1e6
    got = out[sample].float().cpu().numpy()
    err = float(np.abs(got - ref_out).max())
    ok = bool(np.allclose(got, ref_out, atol=1e-2, rtol=1e-2))
    log(f"cpu baseline: {len(sample)} of {B} requests in {t:.2f}s on {threads} threads -> "
        f"{cpu_us / 1e3:.1f} ms per full step; spot check max-abs {err:.2e} "
        f"{'ok' if ok else 'FAILED'}")
    if not ok:
        raise SystemExit("spot check of the GPU output against the oracle failed")
    return {"value": round(cpu_us, 1), "unit": "us", "cores": threads, "kind": "port",
            "sample": f"requests {sample[0]}..{sample[-1]} ({len(sample)} of {B}, "
                      f"{tokens} tokens = {frac * 100:.1f}% of the step), median of 3 runs of "
                      f"oracle/gqa_decode_oracle.c, scaled to the full step",
            "speedup_gpu_vs_cpu": round(cpu_us / gpu_us, 1),
            "spot_check_max_abs": err}


if __name__ == "__main__":
    sys.exit(main())
