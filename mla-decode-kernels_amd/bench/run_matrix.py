"""64-cell benchmark matrix on MI355X: the gfx950 kernels beside a library
baseline, cell by cell comparable with the reference's H100 matrix.

Counterpart of the reference's bench/run_matrix.py:34-175. Grid: headtype
{(32,8),(64,8)} x S {512,2048,8192,32768} x B {1,8,32,128} x block {16,64}.
Per cell (uniform lengths, q/k/v = 0.5 * N(0,1) bf16 from seed 0, shuffled
pool of 1.1x the needed blocks):

* spot check of v1 and of the baseline on the first two requests against an
  fp32 torch reference (atol = rtol = 2e-2);
* median time (HIP events around each call, bench/common.py:49-64 of the
  reference) of the baseline's run() only, v1, v2 at num_splits
  {1,4,8,16,32,64} (best recorded), v2's automatic choice (num_splits=0: the
  token-balanced launch or the split heuristic's count, recorded), the
  token-balanced launch itself (every headtype of the grid), and v0 where it
  is not prohibitively slow (S <= 2048 and B <= 8);
* 0.5 s of untimed calls (steady clocks), then each variant timed as the
  reference times it -- 10 warmup calls, 50 timed (30 for S=32768, B>=32),
  events around each call, synchronize after each -- in two passes over the
  variants, the second in reverse order, keeping each variant's lower
  median, so that clock drift within the cell does not favour whichever
  variant is measured last. (Cells of a few microseconds sit on the launch
  and power-state floor; their times carry no bandwidth information.)

The baseline is torch SDPA on AOTriton over pages gathered into contiguous
K/V at plan time (baselines/sdpa_adapter.py); with --baseline none it is
skipped. Each cell record is a JSON file in --out-dir (MatrixDir) stamped with
the provenance of the library that ran it (python/provenance.py); cells whose
file exists are not run again, so an interrupted run resumes, and
matrix_summary.csv is rebuilt from all cell files at the end.
"""

import argparse
import csv
import itertools
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
import provenance  # noqa: E402
from binding import (KERNELS, automatic_choice, gqa_decode_balanced,  # noqa: E402
                     gqa_decode_v2)

KERNEL_LIB = os.path.join(os.path.dirname(_HERE), "lib", "libgqa_decode_hip.so")

HEADTYPES = [(32, 8), (64, 8)]
S_LIST = [512, 2048, 8192, 32768]
B_LIST = [1, 8, 32, 128]
BLOCK_LIST = [16, 64]
SPLITS_LIST = [1, 4, 8, 16, 32, 64]
POOL_FACTOR = 1.1
MEM_LIMIT_GIB = 200.0
RAMP_SECONDS = 0.5


def cell_name(Hq, Hkv, S, B, bs):
    return f"cell_{Hq}x{Hkv}_S{S}_B{B}_bs{bs}"


def all_cells():
    return [(Hq, Hkv, S, B, bs) for (Hq, Hkv), S, B, bs
            in itertools.product(HEADTYPES, S_LIST, B_LIST, BLOCK_LIST)]


def memory_precheck(cells, baseline):
    """Refuse to start if the largest cell (pool, plus the baseline's
    contiguous copy) cannot fit."""
    need = max(cases.kv_bytes([S] * B, Hkv) * (POOL_FACTOR + (1 if baseline else 0))
               for _, Hkv, S, B, _ in cells) / 2**30
    total = torch.cuda.get_device_properties(0).total_memory / 2**30
    print(f"memory precheck: largest cell needs ~{need:.1f} GiB, device {total:.1f} GiB",
          flush=True)
    if need > min(MEM_LIMIT_GIB, 0.8 * total):
        raise SystemExit(f"largest cell needs {need:.1f} GiB, over the limit")


def ramp(fn, seconds):
    t_end = time.time() + seconds
    while time.time() < t_end:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()


def make_baseline(name, case, scale):
    if name == "sdpa":
        from baselines.sdpa_adapter import make_sdpa_runner
        return make_sdpa_runner(*case, scale)
    raise ValueError(f"unknown baseline {name!r}")


def run_cell(Hq, Hkv, S, B, bs, baseline, num_cus, warmup=None, runs=None):
    """One cell's record. warmup/runs override the reference's counts (for
    quick checks of the harness; the archived matrix uses the defaults)."""
    scale = 1.0 / math.sqrt(cases.D)
    case = cases.make_case([S] * B, Hq, Hkv, bs, pool_factor=POOL_FACTOR, seed=0, qkv_std=0.5)
    kvb = cases.kv_bytes([S] * B, Hkv)
    sol_ms = cases.sol_us(kvb) / 1e3
    checks = {"v1": cases.spot_check(KERNELS["v1"], case, scale, label="v1")}

    dw, dr = (10, 30) if (S == 32768 and B >= 32) else (10, 50)
    warmup = dw if warmup is None else warmup
    runs = dr if runs is None else runs
    mb = case[3].shape[1]
    choice = automatic_choice(B, Hq, Hkv, bs, mb, num_cus) or "balanced"
    checks["v2_auto"] = cases.spot_check(
        lambda *a: gqa_decode_v2(*a, num_splits=0), case, scale, label="v2 automatic")
    with_balanced = Hq // Hkv <= 16  # the balanced launcher's groups (Hkv = 8 here)
    if with_balanced:
        checks["balanced"] = cases.spot_check(gqa_decode_balanced, case, scale, label="balanced")

    fns = {}
    if baseline != "none":
        run = make_baseline(baseline, case, scale)
        checks[baseline] = cases.spot_check(lambda *a: run(), case, scale, label=baseline)
        fns[baseline] = run
    fns["v1"] = lambda: KERNELS["v1"](*case, scale)
    for ns in SPLITS_LIST:
        fns[f"v2/{ns}"] = (lambda n: lambda: gqa_decode_v2(*case, scale, num_splits=n))(ns)
    fns["v2_auto"] = lambda: gqa_decode_v2(*case, scale, num_splits=0)
    if with_balanced:
        fns["balanced"] = lambda: gqa_decode_balanced(*case, scale)
    if S <= 2048 and B <= 8:
        fns["v0"] = lambda: KERNELS["v0"](*case, scale)

    # Clocks drop while the host builds the case; bring them back up first.
    ramp(fns["v2_auto"], RAMP_SECONDS)
    ms = cases.time_ops_two_pass(fns, warmup, runs)

    def entry(t, **extra):
        return dict(median_ms=t, pct_of_sol=sol_ms / t * 100, **extra)

    results = {}
    if baseline != "none":
        results[baseline] = entry(ms[baseline])
    results["v1"] = entry(ms["v1"])
    by_splits = {ns: ms[f"v2/{ns}"] for ns in SPLITS_LIST}
    best = min(by_splits, key=by_splits.get)
    results["v2"] = entry(by_splits[best], by_splits=by_splits, best_splits=best)
    results["v2_auto"] = entry(ms["v2_auto"], choice=choice)
    if with_balanced:
        results["balanced"] = entry(ms["balanced"])
    if "v0" in ms:
        results["v0"] = entry(ms["v0"])

    return {
        "Hq": Hq, "Hkv": Hkv, "S": S, "B": B, "block": bs,
        "warmup": warmup, "runs": runs, "pool_factor": POOL_FACTOR,
        "timing": "events around each call, sync after each; two passes, lower median",
        "kv_bytes": kvb, "sol_ms": sol_ms, "peak_bytes_per_s": cases.HBM_PEAK_BYTES_PER_S,
        "spot_check": {k: f"passed (max-abs {v:.3e})" for k, v in checks.items()},
        "baseline": baseline,
        "clocks": cases.gpu_clocks(),
        "provenance": provenance.stamp("gqa", KERNEL_LIB),
        "results": results,
    }


# matrix_summary.csv: the reference's columns (headtype .. pct_of_sol), then
# the speed ratio against the cell's baseline (named after it, as the
# reference's ratio_vs_flashinfer is; > 1 is faster than the baseline) and the
# automatic launch's recorded choice.
SUMMARY_COLUMNS = ["headtype", "S", "B", "block", "kernel", "best_splits", "median_ms",
                   "pct_of_sol"]


def summary_rows(cell):
    """One summary row per timed variant of a cell record, in column order."""
    base = cell["results"].get(cell.get("baseline", "none"), {}).get("median_ms")
    for kernel, r in cell["results"].items():
        yield [f"{cell['Hq']}x{cell['Hkv']}", cell["S"], cell["B"], cell["block"], kernel,
               r.get("best_splits", ""), r["median_ms"], r["pct_of_sol"],
               base / r["median_ms"] if base else "", r.get("choice", "")]


class MatrixDir:
    """A matrix run's directory: one JSON record per finished cell, written
    whole (temporary file, then rename) so a killed run never leaves half a
    record, and the summary CSV rebuilt from whatever records exist."""

    def __init__(self, path):
        self.path = path
        os.makedirs(path, exist_ok=True)

    def record_path(self, cell):
        return os.path.join(self.path, f"{cell_name(*cell)}.json")

    def has(self, cell):
        return os.path.exists(self.record_path(cell))

    def save(self, cell, record):
        tmp = self.record_path(cell) + ".tmp"
        with open(tmp, "w") as f:
            json.dump(record, f, indent=2)
        os.replace(tmp, self.record_path(cell))

    def records(self):
        """The finished cells' records, in grid order."""
        for cell in all_cells():
            if self.has(cell):
                with open(self.record_path(cell)) as f:
                    yield json.load(f)

    def write_summary(self):
        records = list(self.records())
        if not records:
            return
        baseline = records[0].get("baseline", "none")
        path = os.path.join(self.path, "matrix_summary.csv")
        with open(path, "w", newline="") as f:
            w = csv.writer(f)
            w.writerow(SUMMARY_COLUMNS + [f"ratio_vs_{baseline}", "choice"])
            n = 0
            for rec in records:
                for row in summary_rows(rec):
                    w.writerow(row)
                    n += 1
        print(f"wrote {path} ({n} rows)", flush=True)


def describe(record, baseline):
    """One progress line's worth of a finished cell."""
    r = record["results"]
    auto = r["v2_auto"]
    text = (f"v2 best {r['v2']['median_ms'] * 1e3:.1f} us (ns={r['v2']['best_splits']}), "
            f"automatic {auto['median_ms'] * 1e3:.1f} us ({auto['choice']}, "
            f"{auto['pct_of_sol']:.1f}% SoL)")
    if baseline in r:
        text += f", {baseline} {r[baseline]['median_ms'] * 1e3:.1f} us"
    return text


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--out-dir", default=None,
                    help="matrix directory (resumed if it exists); default results/matrix_<ts>")
    ap.add_argument("--baseline", default="sdpa", choices=["sdpa", "none"])
    ap.add_argument("--only", default=None,
                    help="comma-separated substrings; run only cells whose name contains one")
    ap.add_argument("--warmup", type=int, default=None,
                    help="warmup calls per variant (default: the reference's 10)")
    ap.add_argument("--runs", type=int, default=None,
                    help="timed calls per variant (default: the reference's 50, 30 for "
                         "S=32768 with B>=32)")
    args = ap.parse_args(argv)

    mdir = MatrixDir(args.out_dir or os.path.join(_HERE, "results",
                                                  time.strftime("matrix_%Y%m%d_%H%M%S")))
    print(f"matrix output dir: {mdir.path}", flush=True)
    grid = all_cells()
    if args.only:
        keys = args.only.split(",")
        grid = [c for c in grid if any(k in cell_name(*c) for k in keys)]
    todo = [c for c in grid if not mdir.has(c)]
    print(f"{len(grid) - len(todo)} of {len(grid)} cells already recorded (kept, not rerun); "
          f"{len(todo)} to run", flush=True)
    if todo:
        memory_precheck(todo, args.baseline != "none")
    num_cus = torch.cuda.get_device_properties(0).multi_processor_count

    t_start = time.time()
    for done, cell in enumerate(todo, 1):
        print(f"[{done}/{len(todo)}] {cell_name(*cell)}: running", flush=True)
        record = run_cell(*cell, args.baseline, num_cus, warmup=args.warmup, runs=args.runs)
        mdir.save(cell, record)
        torch.cuda.empty_cache()
        left = (time.time() - t_start) / done * (len(todo) - done) / 60
        print(f"[{done}/{len(todo)}] {cell_name(*cell)}: {describe(record, args.baseline)}; "
              f"~{left:.1f} min left", flush=True)
    mdir.write_summary()


if __name__ == "__main__":
    main()
