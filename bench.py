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
SWEEP_SPLITS = [1, 2, 4, 8, 16, 32, 64]  # --sweep: BASELINE.json's c2 and c3 sweeps
MLA_NAMES = [f"mla_{k}k{sfx}" for sfx in ("", "_sq2") for k in (4, 8, 16, 32)]
MLA_METRIC = ("median µs, TFLOP/s and GB/s of MLA absorbed decode (FlashMLA's accounting), "
              "b=128 h_q=128 h_kv=1 d=576 dv=512 block=64 varlen")
MFMA_BF16_PEAK = 2.5e15
HBM_PEAK = 8e12


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5"] + MLA_NAMES,
                    help="GQA configs c1..c5, or an MLA decode workload (FlashMLA's rows)")
    ap.add_argument("--causal", action="store_true", help="MLA configs: causal mask")
    ap.add_argument("--kernel", default="v2", choices=["v0", "v1", "v2", "balanced"],
                    help="v2 with --num-splits 0 makes the op's automatic choice (balanced or split)")
    ap.add_argument("--num-splits", type=int, default=0, help="v2 split count (0 = heuristic)")
    ap.add_argument("--sweep", action="store_true",
                    help="also time v2 at each of SWEEP_SPLITS splits, as the step is timed")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="oracle threads (default: OMP_NUM_THREADS, else the CPUs this process "
                         "may use)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--ramp-seconds", type=float, default=0.5,
                    help="untimed steps before the warmup steps, to reach steady clocks")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="instead: time a plain device copy of MIB MiB (torch.neg into a second "
                         "buffer), the known-size kernel that calibrates rocprofv3's "
                         "FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--lib", default=None, metavar="PATH",
                    help="C ABI library the timed launches use (default: the in-tree "
                         "lib/libgqa_decode_hip.so); for profiling a build.py --variant build. "
                         "The torch op, which links the in-tree library, is then not timed")
    ap.add_argument("--stream-probe", action="store_true",
                    help="instead: the streaming-read ceiling of config 2's cache (1 GiB of K+V) "
                         "in the scans' head-strided gather and in whole-slot reads, with "
                         "non-temporal and plain loads (lib/libgqa_stream_probe.so)")
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


def kernel_name(kernel, group, balanced=False, hkv=8, B=1, num_splits=1, s_max=0, cus=0):
    """The dominant kernel of one step, by the launchers' rules
    (csrc/gqa_scan.hpp, csrc/gqa_decode_split.hip): v0's kernel; the
    token-balanced scan (matrix-core over 4 or 8 kv-heads); for split launches
    the matrix-core scan from 5 q-heads per group, and for smaller groups the
    split-range kernel once the split count reaches 4 waves' worth per
    (request, kv-head) of one round of one workgroup per CU, the matrix-core
    scan on grids of fewer workgroups than CUs whose splits are at most 1024
    tokens, else the VALU scan."""
    if kernel == "v0":
        return "gqa_decode_v0_kernel"
    if balanced:
        return ("gqa_decode_balanced_mfma_kernel" if hkv in (4, 8)
                else "gqa_decode_balanced_kernel")
    if group >= 5:
        return "gqa_decode_mfma_kernel"
    pairs = B * hkv
    ns = num_splits if kernel == "v2" else 1
    chunk = (-(-s_max // ns) + 31) // 32 * 32
    if cus > 0 and pairs * ns < cus and chunk <= 1024:
        return "gqa_decode_mfma_kernel"
    if ns >= 2 and cus > 0 and ns >= 4 * (cus // pairs if cus > pairs else 1):
        return "gqa_decode_split_range_kernel"
    return "gqa_decode_scan_kernel"


def provenance_stamp(kind, lib_path):
    """Source hashes of the measured path and of the library that ran it
    (python/provenance.py); warns when the library was built from other
    sources than the tree holds."""
    import provenance

    st = provenance.stamp(kind, os.path.abspath(lib_path))
    if not st["library_matches_sources"]:
        log(f"WARNING: {os.path.relpath(lib_path, REPO_ROOT)} was built from sources "
            f"{st['library_source_sha16']}, the tree holds {st['source_sha16']}: rebuild")
    return st


def ramp(torch, step, seconds, warmup):
    """Clock ramp: the GPU takes a few hundred milliseconds of load to reach
    its steady clocks, far longer than a few short steps; run untimed steps
    for `seconds`, then `warmup` more."""
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(8):
            step()
        torch.cuda.synchronize()
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()


def timed_steps(torch, step, stream, K):
    """Time exactly K calls of step() back to back on `stream`. Events sit only
    between groups of steps (an event between two kernels delays the second
    one), so each group's average is the steady-state step time. Returns the
    median group average (us), the sorted group averages and the wall time (s)."""
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
    return group_us[groups // 2], group_us, wall


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

    if args.lib:
        capi.LIB_PATH = os.path.abspath(args.lib)
        log(f"C ABI library: {capi.LIB_PATH}")
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    props = torch.cuda.get_device_properties(dev)
    if args.stream_probe:
        return stream_probe(torch, cases, dev)
    if args.copy_probe:
        n = args.copy_probe << 20
        x = torch.ones(n // 4, dtype=torch.float32, device=dev)
        y = torch.empty_like(x)
        ms = cases.time_op(lambda: torch.neg(x, out=y), warmup=3, runs=10)
        print(json.dumps({"copy_probe": "torch.neg fp32", "read_bytes": n, "write_bytes": n,
                          "median_us": round(ms * 1e3, 2),
                          "gbps_read_plus_write": round(2 * n / ms / 1e6, 1)}), flush=True)
        return 0
    if args.config in MLA_NAMES:
        return main_mla(args, dev, props)
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
    # v2 with num_splits 0 takes the C ABI's automatic rule: the
    # token-balanced launch where gqa_decode_prefer_balanced says so, else the
    # split heuristic's count. (The torch op also takes one split for block
    # tables of at most 512 tokens, where it allocates the split workspace
    # inside the call; here the workspace is allocated once, as a C ABI
    # caller would, and the heuristic's count is the faster one.)
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

    ramp(torch, step, args.ramp_seconds, args.warmup)

    # Timed region: exactly K steps back to back.
    median_us, group_us, wall = timed_steps(torch, step, stream, args.steps)
    K = args.steps

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

    # The torch operator, timed the reference's way (not for a --lib variant:
    # the op runs the in-tree library).
    op_ms = None
    if not args.lib:
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
        # v2 at each split count, timed as the step above: partial + merge
        # launches through the C ABI (one launch for one split) with a
        # caller-owned workspace, K steps back to back after a warmup.
        sweep = {}
        top = max(SWEEP_SPLITS)
        ws_s = torch.empty(B * Hq * top * (cases.D + 2), dtype=torch.float32, device=dev)
        for s in SWEEP_SPLITS:
            st = B * Hq * s
            acc_s, m_s, l_s = (ws_s.data_ptr(), ws_s.data_ptr() + st * cases.D * 4,
                               ws_s.data_ptr() + st * (cases.D + 1) * 4)

            def sweep_step(s=s, acc_s=acc_s, m_s=m_s, l_s=l_s):
                if capi.v2_launch(*ptrs, out.data_ptr(), B, Hq, Hkv, bs, mb, scale, s, acc_s,
                                  m_s, l_s, sp) != 0:
                    raise RuntimeError(f"v2 launch failed at num_splits={s}")

            def sweep_partial(s=s, acc_s=acc_s, m_s=m_s, l_s=l_s):
                if capi.v2_partial_launch(*ptrs, B, Hq, Hkv, bs, mb, scale, s, acc_s, m_s, l_s,
                                          sp) != 0:
                    raise RuntimeError(f"v2 partial launch failed at num_splits={s}")
            ramp(torch, sweep_step, args.ramp_seconds, args.warmup)
            us = timed_steps(torch, sweep_step, stream, K)[0]
            part_us = timed_steps(torch, sweep_partial, stream, K)[0]
            sweep[s] = {"us": round(us, 2), "pct_of_sol": round(sol / us * 100, 2),
                        "partial_us": round(part_us, 2)}
            log(f"  sweep num_splits={s}: {us:.2f} us ({sol / us * 100:.1f}% SoL), "
                f"partial kernel {part_us:.2f} us")

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
        "config": {"workload": f"{args.config}: {cfg['desc']}" + (
                       f" [library {os.path.relpath(capi.LIB_PATH, REPO_ROOT)}]" if args.lib else ""),
                   "Hq": Hq, "Hkv": Hkv, "B": B,
                   "S": cfg["S"] if cfg["S"] else "U[1,32768]", "block": bs,
                   "kernel": args.kernel,
                   "num_splits": split_label if args.kernel in ("v2", "balanced") else None},
        "pct_of_sol": round(sol / median_us * 100, 2),
        "achieved_gbps": round(kvb / median_us / 1e3, 1),
        "kv_bytes": kvb,
        "sol_us": round(sol, 3),
        "op_median_us": round(op_ms * 1e3, 3) if op_ms is not None else None,
        "roofline": {"bound": "hbm",
                     "kernel": kernel_name(args.kernel, Hq // Hkv, balanced, Hkv, B,
                                           ns if not balanced else 1, mb * bs,
                                           props.multi_processor_count),
                     "achieved": round(achieved, 1),
                     "peak": 8000.0, "unit": "GB/s", "frac": round(achieved / 8000.0, 4),
                     "avg_kernel_us": round(kern_avg_us, 3),
                     "traffic": traffic},
        "device": props.name, "gcn_arch": props.gcnArchName, "cus": props.multi_processor_count,
        "clocks": cases.gpu_clocks(),
        "provenance": provenance_stamp("gqa", capi.LIB_PATH),
    }
    if sweep:
        result["sweep_us"] = sweep

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args, case, out, S_list, scale, median_us)
    print(json.dumps(result), flush=True)
    return 0


def main_mla(args, dev, props):
    """One MLA decode step over a FlashMLA benchmark workload, timed as the GQA
    steps are: the token-balanced launch (plan, split and merge kernels; one
    workgroup per CU) by default, or with --num-splits N the fixed-split
    launch (split kernel, then the combine kernel when N > 1)."""
    import torch

    import capi
    import cases

    cfg = cases.MLA_CONFIGS[args.config]
    B, s_q, h_q, bs = cfg["B"], cfg["s_q"], cfg["h_q"], cfg["bs"]
    S_list = cases.mla_seq_lens(B, cfg["S_mean"], args.seed, s_q)
    flops, nbytes = cases.mla_flops_bytes(S_list, s_q, h_q)
    ridge = MFMA_BF16_PEAK / HBM_PEAK
    bound = "mfma" if flops / nbytes > ridge else "hbm"
    sol = max(flops / MFMA_BF16_PEAK, nbytes / HBM_PEAK) * 1e6
    log(f"config {args.config}: B={B} s_q={s_q} h_q={h_q} sum(S)={sum(S_list)}; "
        f"{flops / 1e9:.1f} GFLOP, {nbytes / 1e6:.1f} MB; {bound}-bound, SoL {sol:.1f} us")
    t0 = time.time()
    case = cases.make_mla_case(S_list, s_q, h_q, bs, seed=args.seed, device=dev)
    q, kv, bt, sl = case
    torch.cuda.synchronize()
    log(f"inputs resident in HBM ({time.time() - t0:.1f}s)")
    mb = bt.shape[1]
    scale = 576 ** -0.5
    cus = props.multi_processor_count
    balanced = args.num_splits == 0
    ns = args.num_splits
    out = torch.empty(B, s_q, h_q, 512, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(B, h_q, s_q, dtype=torch.float32, device=dev)
    wsb = (capi.mla_balanced_workspace_bytes(B, s_q, h_q, cus) if balanced
           else capi.mla_workspace_bytes(B, s_q, h_q, ns))
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    largs = (q.data_ptr(), kv.data_ptr(), bt.data_ptr(), sl.data_ptr(), out.data_ptr(),
             lse.data_ptr(), B, s_q, h_q, bs, mb, scale, int(args.causal),
             cus if balanced else ns, ws.data_ptr(), wsb, sp)
    launch = capi.mla_balanced_launch if balanced else capi.mla_launch

    def step():
        rc = launch(*largs)
        if rc != 0:
            raise RuntimeError(f"MLA launch failed: hipError_t {rc}")

    t_ramp = time.perf_counter() + args.ramp_seconds
    while time.perf_counter() < t_ramp:
        for _ in range(4):
            step()
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

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

    # The split kernel alone, K launches back to back: its average duration
    # (fixed splits; the balanced split kernel needs its plan launch first, so
    # there the whole step stands in, and the rocprofv3 summary splits it).
    if balanced:
        kern_us = median_us
    else:
        kev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        kev[0].record(stream)
        for _ in range(K):
            if capi.mla_splitkv_launch(*largs) != 0:
                raise RuntimeError("mla_decode_splitkv_launch failed")
        kev[1].record(stream)
        torch.cuda.synchronize()
        kern_us = kev[0].elapsed_time(kev[1]) * 1e3 / K
    step()  # out and lse of a whole step again, for the spot check
    torch.cuda.synchronize()
    tflops_k = flops / kern_us / 1e6
    gbps_k = nbytes / kern_us / 1e3
    log(f"mla: median step {median_us:.2f} us (groups {group_us[0]:.1f}..{group_us[-1]:.1f}), "
        f"split kernel avg {kern_us:.2f} us ({tflops_k:.0f} TFLOP/s, {gbps_k:.0f} GB/s), "
        f"{'balanced' if balanced else f'num_splits {ns}'}")
    achieved = tflops_k if bound == "mfma" else gbps_k
    peak = MFMA_BF16_PEAK / 1e12 if bound == "mfma" else HBM_PEAK / 1e9
    h100 = cases.MLA_H100_MS.get(args.config)
    result = {
        "metric": MLA_METRIC,
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
        "config": {"workload": f"{args.config}: FlashMLA row b={B} s_q={s_q} "
                               f"s_k={cfg['S_mean']} varlen h_q={h_q} h_kv=1 block={bs}",
                   "causal": bool(args.causal),
                   "launch": "balanced" if balanced else f"num_splits={ns}"},
        "tflops": round(flops / median_us / 1e6, 1),
        "gbps": round(nbytes / median_us / 1e3, 1),
        "flops": flops, "bytes": nbytes,
        "pct_of_sol": round(sol / median_us * 100, 2),
        "flashmla_h100_us": h100 * 1e3 if h100 else None,
        "roofline": {"bound": bound,
                     "kernel": "whole step" if balanced else "mla_decode_kernel",
                     "achieved": round(achieved, 1),
                     "peak": peak, "unit": "TFLOP/s" if bound == "mfma" else "GB/s",
                     "frac": round(achieved / peak, 4), "avg_kernel_us": round(kern_us, 3),
                     "mfma_frac": round(tflops_k * 1e12 / MFMA_BF16_PEAK, 4),
                     "hbm_frac": round(gbps_k * 1e9 / HBM_PEAK, 4),
                     "traffic": read_traffic(args.config, "mla", "balanced" if balanced else ns)},
        "device": props.name, "gcn_arch": props.gcnArchName, "cus": props.multi_processor_count,
        "clocks": cases.gpu_clocks(),
        "provenance": provenance_stamp("mla", capi.LIB_PATH),
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline_mla(args, case, out, lse, S_list, scale, median_us)
    print(json.dumps(result), flush=True)
    return 0


def stream_probe(torch, cases, dev):
    """Read rate of config 2's K and V (32 requests x 8192 token slots x 8
    kv-heads x 256 B each: 1 GiB together), every byte once, no arithmetic:
    the scans' head-strided gather (one workgroup of 4 waves per (kv-head,
    request), as the VALU scan runs config 2 at one split), whole-slot reads
    (4 waves per (request, split), 8 splits) and a plain linear read of both
    buffers (256 workgroups of 4 waves), each with non-temporal and plain
    loads. Events around each launch, median of 20 after 5 warmup launches.
    Then the timed launches (non-temporal): the head-strided gather and a
    dynamic one (256 persistent workgroups claiming items of 512 or 1024 token
    slots of one (request, kv-head)), with each workgroup's end time on the
    GPU's 100 MHz real-time counter (from the launch's first start, last of
    the 20 timed launches): how much of a launch is its tail. Between the
    two, grids of 64 and 128 workgroups (the ceiling of launches that leave
    CUs idle) and the head-strided read through a block table of 16-slot
    blocks, identity and shuffled (config 2's access pattern)."""
    import ctypes

    path = os.path.join(PKG_DIR, "lib", "libgqa_stream_probe.so")
    if not os.path.exists(path):
        raise SystemExit(f"{path} missing: run `python mla-decode-kernels_amd/build.py`")
    L = ctypes.CDLL(path)
    L.gqa_stream_probe_launch.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int] * 5 + [
        ctypes.c_void_p]
    L.gqa_stream_probe_launch.restype = ctypes.c_int
    requests, slots, splits = 32, 8192, 8
    nbytes = requests * slots * 2048
    k = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    v = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    k.random_(0, 256)
    v.random_(0, 256)
    sink = torch.empty(max(requests * 8 * 256, 128 * 1024), dtype=torch.int32, device=dev)
    sp = torch.cuda.current_stream().cuda_stream
    res = {}
    for pattern, pname, nsplit in ((0, "head_strided", 1), (1, "whole_slot", splits),
                                   (2, "linear", 256)):
        for nt in (1, 0):
            def launch():
                rc = L.gqa_stream_probe_launch(k.data_ptr(), v.data_ptr(), sink.data_ptr(),
                                               pattern, requests, slots, nsplit, nt, sp)
                if rc != 0:
                    raise RuntimeError(f"gqa_stream_probe_launch returned {rc}")
            ms = cases.time_op(launch, warmup=5, runs=20)
            if pattern == 0 and nt:
                folds = sink[:requests * 8 * 256].clone()  # the paged reads' check below
            key = f"{pname}_{'nt' if nt else 'plain'}"
            res[key] = {"median_us": round(ms * 1e3, 2),
                        "tbps": round(2 * nbytes / ms / 1e9, 3),
                        "frac_of_8tbps": round(2 * nbytes / ms / 1e9 / 8.0, 4)}
            log(f"stream probe {key}: {ms * 1e3:.2f} us, {2 * nbytes / ms / 1e9:.3f} TB/s")
    # Grids that occupy only part of the CUs: what 64 or 128 CUs stream on
    # their own (linear, 4 or 16 waves per workgroup), and config 3's gather
    # at one split (8 requests x 32768 slots: grid (8 kv-heads, 8 requests),
    # 64 workgroups of 4 waves) and at two (each request's halves as 16
    # requests of 16384 slots: 128 workgroups) over the same bytes.
    for pattern, pname, reqs, sl, nsplit in ((2, "linear_64wg_4w", requests, slots, 64),
                                            (4, "linear_64wg_16w", requests, slots, 64),
                                            (2, "linear_128wg_4w", requests, slots, 128),
                                            (4, "linear_128wg_16w", requests, slots, 128),
                                            (0, "head_strided_c3_1split", 8, 32768, 1),
                                            (0, "head_strided_c3_2split", 16, 16384, 1)):
        def launch():
            rc = L.gqa_stream_probe_launch(k.data_ptr(), v.data_ptr(), sink.data_ptr(), pattern,
                                           reqs, sl, nsplit, 1, sp)
            if rc != 0:
                raise RuntimeError(f"gqa_stream_probe_launch returned {rc}")
        ms = cases.time_op(launch, warmup=3, runs=10)
        res[pname] = {"median_us": round(ms * 1e3, 2), "tbps": round(2 * nbytes / ms / 1e9, 3),
                      "frac_of_8tbps": round(2 * nbytes / ms / 1e9 / 8.0, 4)}
        log(f"stream probe {pname}: {ms * 1e3:.2f} us, {2 * nbytes / ms / 1e9:.3f} TB/s")
    # The head-strided read through a block table of 16-slot blocks, as
    # config 2's cache is read: an identity table (the pattern above, with the
    # scalar block-id loads) and config 2's seeded shuffle of the pool.
    L.gqa_stream_probe_paged_launch.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 2 + [
        ctypes.c_void_p]
    L.gqa_stream_probe_paged_launch.restype = ctypes.c_int
    nblk = slots // 16
    perm = torch.randperm(requests * nblk, generator=torch.Generator().manual_seed(0))
    for pname, table in (("paged_identity", torch.arange(requests * nblk)), ("paged_shuffled", perm)):
        bt = table.to(torch.int32).view(requests, nblk).to(dev)
        def launch():
            rc = L.gqa_stream_probe_paged_launch(k.data_ptr(), v.data_ptr(), bt.data_ptr(),
                                                 sink.data_ptr(), requests, nblk, sp)
            if rc != 0:
                raise RuntimeError(f"gqa_stream_probe_paged_launch returned {rc}")
        ms = cases.time_op(launch, warmup=5, runs=20)
        # Every lane sums its loads' folds: through the identity table each
        # lane reads what it reads in the head-strided pattern, and through
        # the shuffled one the lanes' sum over the grid is the same sum, if
        # every 16 bytes of both pools are read exactly once.
        got = sink[:requests * 8 * 256]
        if pname == "paged_identity" and not torch.equal(got, folds):
            raise RuntimeError("paged probe (identity table) read other bytes than head-strided")
        if (int(got.to(torch.int64).sum()) - int(folds.to(torch.int64).sum())) % 2**32:
            raise RuntimeError(f"{pname}: the pools were not read exactly once")
        res[pname] = {"median_us": round(ms * 1e3, 2), "tbps": round(2 * nbytes / ms / 1e9, 3),
                      "frac_of_8tbps": round(2 * nbytes / ms / 1e9 / 8.0, 4)}
        log(f"stream probe {pname}: {ms * 1e3:.2f} us, {2 * nbytes / ms / 1e9:.3f} TB/s")
    L.gqa_stream_probe_timed_launch.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 4 + [
        ctypes.c_void_p]
    L.gqa_stream_probe_timed_launch.restype = ctypes.c_int
    times = torch.zeros(2 * max(8 * requests, 256), dtype=torch.int64, device=dev)
    ctr = torch.zeros(2, dtype=torch.int32, device=dev)
    for pattern, pname, chunk in ((0, "timed_head_strided", 0), (3, "dynamic_512", 512),
                                  (3, "dynamic_1024", 1024)):
        def launch():
            rc = L.gqa_stream_probe_timed_launch(k.data_ptr(), v.data_ptr(), sink.data_ptr(),
                                                 times.data_ptr(), ctr.data_ptr(), pattern,
                                                 requests, slots, chunk, sp)
            if rc != 0:
                raise RuntimeError(f"gqa_stream_probe_timed_launch returned {rc}")
        ms = cases.time_op(launch, warmup=5, runs=20)
        nwg = 8 * requests if pattern == 0 else 256
        t = times[:2 * nwg].view(nwg, 2).cpu().double()
        ends = sorted(((t[:, 1] - t[:, 0].min()) * 0.01).tolist())  # 100 MHz ticks -> us
        q = lambda f: round(ends[min(int(f * nwg), nwg - 1)], 2)  # noqa: E731
        res[pname] = {"median_us": round(ms * 1e3, 2), "tbps": round(2 * nbytes / ms / 1e9, 3),
                      "wg_end_us": {"min": round(ends[0], 2), "p10": q(0.1), "p50": q(0.5),
                                    "p90": q(0.9), "max": round(ends[-1], 2)}}
        log(f"stream probe {pname}: {ms * 1e3:.2f} us; workgroup ends (us) min {ends[0]:.1f} "
            f"p50 {q(0.5)} max {ends[-1]:.1f}")
    if int(ctr.abs().sum()) != 0:
        raise RuntimeError("dynamic probe left its counters non-zero")
    print(json.dumps({"stream_probe": "config 2 cache, 1 GiB K+V, identity block table",
                      "bytes": 2 * nbytes, "results": res, "clocks": cases.gpu_clocks()}),
          flush=True)
    return 0


def cpu_threads(args):
    """(threads, source) for the CPU baseline: --cpu-threads if given, else this
    process's CPU share -- OMP_NUM_THREADS where the host sets it (the GPU
    boxes set it to their per-GPU share, 16, whatever os.cpu_count() reports),
    capped at the CPUs the process may run on."""
    avail = len(os.sched_getaffinity(0))
    if args.cpu_threads:
        return args.cpu_threads, "--cpu-threads"
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        return min(int(omp), avail), "OMP_NUM_THREADS"
    return avail, "sched_getaffinity"


def host_cpu_record(threads, source):
    return {"cores": threads, "threads_from": source, "host_cpu_count": os.cpu_count(),
            "affinity_cpus": len(os.sched_getaffinity(0))}


def cpu_baseline_mla(args, case, out, lse, S_list, scale, gpu_us):
    """The MLA oracle (oracle/mla_decode_oracle.c) on this host's cores over
    whole requests of the workload (~10 s per run), run until ~10 s of CPU
    time has been timed (at least 3 runs), the median run scaled to one full
    step; its output on the sample is compared with the GPU's (out within
    2e-2, lse 5e-3)."""
    import numpy as np

    from cases import mla_host_case
    sys.path.insert(0, REPO_ROOT)
    from oracle import c_oracle  # noqa: E402  (the checker, timed as the CPU baseline)

    threads, source = cpu_threads(args)
    B = len(S_list)
    t0 = time.perf_counter()
    c_oracle.mla_decode_ref(*mla_host_case(case, [0]), scale, causal=args.causal,
                            nthreads=threads)
    per_token = (time.perf_counter() - t0) / max(S_list[0], 1)
    budget_s, sample, tokens = 10.0, [], 0
    for b in range(B):
        if sample and (tokens + S_list[b]) * per_token > budget_s:
            break
        sample.append(b)
        tokens += S_list[b]
    hc = mla_host_case(case, sample)
    times = []
    while len(times) < 3 or (sum(times) < budget_s and len(times) < 1000):
        t0 = time.perf_counter()
        ref_out, ref_lse = c_oracle.mla_decode_ref(*hc, scale, causal=args.causal,
                                                   nthreads=threads)
        times.append(time.perf_counter() - t0)
    t = sorted(times)[len(times) // 2]
    frac = tokens / sum(S_list)
    cpu_us = t / frac * 1e6
    got = out[sample].float().cpu().numpy()
    got_lse = lse[sample].cpu().numpy()
    err = float(np.abs(got - ref_out).max())
    lse_err = float(np.abs(got_lse - ref_lse).max())
    ok = bool(np.allclose(got, ref_out, atol=2e-2, rtol=2e-2)) and lse_err <= 5e-3
    log(f"cpu baseline: {len(sample)} of {B} requests in {t:.2f}s on {threads} threads -> "
        f"{cpu_us / 1e3:.1f} ms per full step; spot check max-abs {err:.2e}, lse {lse_err:.2e} "
        f"{'ok' if ok else 'FAILED'}")
    if not ok:
        raise SystemExit("spot check of the GPU output against the oracle failed")
    return {"value": round(cpu_us, 1), "unit": "us", **host_cpu_record(threads, source),
            "kind": "port",
            "sample": f"requests {sample[0]}..{sample[-1]} ({len(sample)} of {B}, "
                      f"{tokens} tokens = {frac * 100:.1f}% of the step), median of "
                      f"{len(times)} runs ({sum(times):.1f} s) of oracle/mla_decode_oracle.c, "
                      f"scaled to the full step",
            "speedup_gpu_vs_cpu": round(cpu_us / gpu_us, 1),
            "spot_check_max_abs": err, "spot_check_lse_max_abs": lse_err}


def cpu_baseline(args, case, out, S_list, scale, gpu_us):
    """The oracle on this host's cores over a bounded sample of the workload
    (whole requests, at most ~10 s per run), run until ~10 s of CPU time has
    been timed (at least 3 runs), the median run scaled to one full step."""
    import numpy as np

    from cases import host_case
    sys.path.insert(0, REPO_ROOT)
    from oracle import c_oracle  # noqa: E402  (the checker, timed as the CPU baseline)

    threads, source = cpu_threads(args)
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
    while len(times) < 3 or (sum(times) < budget_s and len(times) < 1000):
        t0 = time.perf_counter()
        ref_out = c_oracle.attention_ref(*hc, scale, nthreads=threads)
        times.append(time.perf_counter() - t0)
    t = sorted(times)[len(times) // 2]
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
    return {"value": round(cpu_us, 1), "unit": "us", **host_cpu_record(threads, source),
            "kind": "port",
            "sample": f"requests {sample[0]}..{sample[-1]} ({len(sample)} of {B}, "
                      f"{tokens} tokens = {frac * 100:.1f}% of the step), median of "
                      f"{len(times)} runs ({sum(times):.1f} s) of oracle/gqa_decode_oracle.c, "
                      f"scaled to the full step",
            "speedup_gpu_vs_cpu": round(cpu_us / gpu_us, 1),
            "spot_check_max_abs": err}


if __name__ == "__main__":
    sys.exit(main())
