"""rocprofv3 passes over one bench.py configuration, and their summary.

The MI355X counterpart of the reference's analysis/ncu/run_ncu.sh and
extract.py (Nsight Compute sections reduced to DRAM bytes, L2 hit,
occupancy, stalls): one rocprofv3 run per pass, each under its own time limit,
then a reduction of the CSV output to per-kernel durations, per-kernel
counter means and the HBM traffic of the dominant kernel, calibrated by the
same counters on a plain 1 GiB copy (bench.py --copy-probe 1024).

    python profile_config.py --config c5 --out-dir <dir>          # run + summarize
    python profile_config.py --summarize <dir> [--config c5]      # summarize only
    ... --profile-md profiles/<name>.md   # also write the complete profile file

Passes (each counter set within one rocprofv3 pass's hardware limits):
  trace   --kernel-trace --stats over a 50-step bench run
  fetch   FETCH_SIZE                     write   WRITE_SIZE
  occ     SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_ACTIVE_INST_VALU SQ_VALU_MFMA_BUSY_CYCLES
          SQ_WAIT_INST_ANY SQ_INSTS_VALU SQ_INSTS_MFMA GRBM_GUI_ACTIVE
  lds     SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_INSTS_LDS SQ_WAVES SQ_INSTS_VMEM_RD
          GRBM_GUI_ACTIVE
  l2      TCC_HIT_sum TCC_MISS_sum
  stall   SQ_WAVE_CYCLES SQ_WAIT_ANY SQ_WAIT_INST_ANY SQ_ACTIVE_INST_VALU
          SQ_ACTIVE_INST_VMEM SQ_ACTIVE_INST_LDS SQ_ACTIVE_INST_SCA SQ_ACTIVE_INST_MISC
  copy_fetch / copy_write   the copy calibration (FETCH_SIZE / WRITE_SIZE)
This script never touches the GPU itself: rocprofv3 starts bench.py as its
program (after `--`), one child process per pass. --bench-args adds bench.py
arguments to every pass but the copies (e.g. "--num-splits 4", or "--lib
<path>" to profile a library built with build.py --variant).

The summary also gives, per kernel, the counterparts of the reference
extractor's stall and occupancy sections (analysis/ncu/extract.py:126-191):
  wave-cycle breakdown  the stall pass's counters as fractions of
      SQ_WAVE_CYCLES (all in quad-cycles): waiting on a dependency
      (SQ_WAIT_ANY: s_waitcnt on memory, LDS or a previous result), waiting
      for issue (SQ_WAIT_INST_ANY: ready, but the SIMD issued another wave's
      instruction or the unit was busy), and issuing each instruction type
      (SQ_ACTIVE_INST_*); the three largest are listed as the top reasons;
  occupancy limiter     waves per SIMD allowed by each resource of the
      dispatch (VGPRs + AGPRs per lane out of 512 in granules of 8, LDS per
      workgroup out of 160 KiB, 8 waves per SIMD, and the grid itself),
      from the kernel-trace columns; the smallest is the limiter.
"""

import argparse
import csv
import glob
import json
import os
import re
import statistics
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO_ROOT = os.path.dirname(os.path.dirname(HERE))
BENCH = os.path.join(REPO_ROOT, "bench.py")
COPY_BYTES = 1 << 30

PASSES = {
    "trace": ["--kernel-trace", "--stats"],
    "fetch": ["--pmc", "FETCH_SIZE"],
    "write": ["--pmc", "WRITE_SIZE"],
    "occ": ["--pmc", "SQ_WAVE_CYCLES", "SQ_BUSY_CYCLES", "SQ_ACTIVE_INST_VALU",
            "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_WAIT_INST_ANY", "SQ_INSTS_VALU", "SQ_INSTS_MFMA",
            "GRBM_GUI_ACTIVE"],
    "lds": ["--pmc", "SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE", "SQ_INSTS_LDS", "SQ_WAVES",
            "SQ_INSTS_VMEM_RD", "GRBM_GUI_ACTIVE"],
    "l2": ["--pmc", "TCC_HIT_sum", "TCC_MISS_sum"],
    "stall": ["--pmc", "SQ_WAVE_CYCLES", "SQ_WAIT_ANY", "SQ_WAIT_INST_ANY", "SQ_ACTIVE_INST_VALU",
              "SQ_ACTIVE_INST_VMEM", "SQ_ACTIVE_INST_LDS", "SQ_ACTIVE_INST_SCA",
              "SQ_ACTIVE_INST_MISC"],
    "copy_fetch": ["--pmc", "FETCH_SIZE"],
    "copy_write": ["--pmc", "WRITE_SIZE"],
}
SHORT_RUN = ["--steps", "3", "--warmup", "1", "--ramp-seconds", "0", "--no-cpu-baseline"]


def bench_args(pass_name, config, extra=()):
    extra = list(extra)
    if "--lib" in extra:  # the passes run from /tmp: a library path is taken from the repo root
        i = extra.index("--lib") + 1
        extra[i] = os.path.join(REPO_ROOT, extra[i])
    if pass_name.startswith("copy_"):
        return ["--copy-probe", "1024"]
    if pass_name == "trace":
        return ["--config", config, "--steps", "50", "--no-cpu-baseline"] + list(extra)
    return ["--config", config] + SHORT_RUN + list(extra)


def command(pass_name, config, out_dir, extra=()):
    return (["rocprofv3", "-f", "csv"] + PASSES[pass_name] +
            ["-d", os.path.join(out_dir, pass_name), "-o", "run", "--", sys.executable, BENCH] +
            bench_args(pass_name, config, extra))


def run_passes(config, out_dir, passes, timeout, extra=()):
    os.makedirs(out_dir, exist_ok=True)
    env = dict(os.environ, TMPDIR="/tmp")
    for name in passes:
        cmd = command(name, config, out_dir, extra)
        print("==", name, " ".join(cmd), flush=True)
        with open(os.path.join(out_dir, f"{name}.log"), "w") as log:
            # A pass that asks for more counters than the hardware holds hangs
            # instead of failing; the limit ends it (and the script).
            proc = subprocess.run(cmd, cwd="/tmp", env=env, stdout=log, stderr=subprocess.STDOUT,
                                  timeout=timeout)
        if proc.returncode != 0:
            raise SystemExit(f"pass {name} failed with status {proc.returncode}")
        for db in glob.glob(os.path.join(out_dir, name, "**", "*.db"), recursive=True):
            os.remove(db)  # raw databases stay out of the summary folder


# ------------------------------------------------------------------ summary

def short_name(name):
    """Kernel name without its argument list, 'void ' prefix and anonymous
    namespace qualifier."""
    name = name.replace("(anonymous namespace)::", "")
    return re.sub(r"\(.*", "", name).replace("void ", "").strip()


def read_csvs(directory, suffix):
    rows = []
    for f in sorted(glob.glob(os.path.join(directory, "**", f"*{suffix}"), recursive=True)):
        with open(f) as fh:
            rows.extend(csv.DictReader(fh))
    return rows


MLA_CONFIGS = [f"mla_{k}k{sfx}" for sfx in ("", "_sq2") for k in (4, 8, 16, 32)]


def kernel_durations(directory, pattern="gqa|mla"):
    """{kernel: [durations in us]} from a --kernel-trace pass."""
    out = {}
    for r in read_csvs(directory, "kernel_trace.csv"):
        name = r.get("Kernel_Name", "")
        if re.search(pattern, name):
            dt = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            out.setdefault(short_name(name), []).append(dt)
    return out


def counter_means(directory, pattern="gqa|mla|neg_kernel"):
    """{(kernel, counter): mean value over dispatches} from a --pmc pass."""
    acc = {}
    for r in read_csvs(directory, "counter_collection.csv"):
        name = r.get("Kernel_Name", "")
        if re.search(pattern, name):
            acc.setdefault((short_name(name), r["Counter_Name"]), []).append(
                float(r["Counter_Value"]))
    return {k: sum(v) / len(v) for k, v in acc.items()}


STALL_PARTS = [("dependency wait", "SQ_WAIT_ANY"), ("issue wait", "SQ_WAIT_INST_ANY"),
               ("VALU/MFMA issue", "SQ_ACTIVE_INST_VALU"), ("VMEM issue", "SQ_ACTIVE_INST_VMEM"),
               ("LDS issue", "SQ_ACTIVE_INST_LDS"), ("scalar issue", "SQ_ACTIVE_INST_SCA"),
               ("branch/message", "SQ_ACTIVE_INST_MISC")]


def stall_breakdown(counters, kernel):
    """[(label, fraction of SQ_WAVE_CYCLES)] for one kernel, largest first, or
    None without the stall pass."""
    total = counters.get((kernel, "SQ_WAVE_CYCLES"))
    if not total:
        return None
    parts = [(label, counters[(kernel, c)] / total) for label, c in STALL_PARTS
             if (kernel, c) in counters]
    return sorted(parts, key=lambda p: -p[1])


LDS_BYTES_PER_CU = 160 * 1024
VGPRS_PER_SIMD_LANE = 512
MAX_WAVES_PER_SIMD = 8


def occupancy(row, num_cus=256):
    """({resource: waves per SIMD it allows}, limiter) for one kernel-trace row."""
    wg = int(row["Workgroup_Size_X"]) * int(row["Workgroup_Size_Y"]) * int(row["Workgroup_Size_Z"])
    waves_per_wg = -(-wg // 64)
    vgprs = int(row.get("VGPR_Count") or 0) + int(row.get("Accum_VGPR_Count") or 0)
    lds = int(row.get("LDS_Block_Size") or 0)
    grid = int(row["Grid_Size_X"]) * int(row["Grid_Size_Y"]) * int(row["Grid_Size_Z"])
    limits = {"max waves": MAX_WAVES_PER_SIMD}
    if vgprs:
        limits["VGPRs"] = VGPRS_PER_SIMD_LANE // (-(-vgprs // 8) * 8)
    if lds:
        wgs = LDS_BYTES_PER_CU // lds
        limits["LDS"] = wgs * waves_per_wg / 4
    limits["grid"] = grid / 64 / (num_cus * 4)
    limiter = min(limits, key=limits.get)
    return limits, limiter


def occupancy_rows(directory, pattern="gqa|mla|probe"):
    """{kernel: first kernel-trace row} (the resource columns are per kernel)."""
    out = {}
    for r in read_csvs(directory, "kernel_trace.csv"):
        name = r.get("Kernel_Name", "")
        if re.search(pattern, name) and r.get("Workgroup_Size_X"):
            out.setdefault(short_name(name), r)
    return out


def calibration(root):
    """Bytes per counter unit for FETCH_SIZE and WRITE_SIZE: the copy of
    COPY_BYTES read and written, over what each counter reported for it."""
    f = {k: v for k, v in counter_means(os.path.join(root, "copy_fetch"), "neg_kernel").items()
         if k[1] == "FETCH_SIZE"}
    w = {k: v for k, v in counter_means(os.path.join(root, "copy_write"), "neg_kernel").items()
         if k[1] == "WRITE_SIZE"}
    if len(f) != 1 or len(w) != 1:
        return None
    return COPY_BYTES / next(iter(f.values())), COPY_BYTES / next(iter(w.values()))


def coalescing(counters, cal):
    """[(kernel, HBM bytes fetched, VMEM read instructions, bytes per
    instruction, L2 hit rate or None)] for kernels with both counters."""
    if not cal:
        return []
    rows = []
    for (k, c), v in sorted(counters.items()):
        insts = counters.get((k, "SQ_INSTS_VMEM_RD"))
        if c != "FETCH_SIZE" or not insts:
            continue
        fetched = v * cal[0]
        hit, miss = counters.get((k, "TCC_HIT_sum")), counters.get((k, "TCC_MISS_sum"))
        rate = hit / (hit + miss) if hit is not None and miss is not None and hit + miss else None
        rows.append((k, fetched, insts, fetched / insts, rate))
    return rows


def summarize(root):
    lines = []
    dur = kernel_durations(os.path.join(root, "trace"))
    lines.append("| kernel | calls | average | median | min | max | std dev |")
    lines.append("|---|---|---|---|---|---|---|")
    for name, v in sorted(dur.items(), key=lambda kv: -sum(kv[1])):
        v = sorted(v)
        sd = statistics.pstdev(v) if len(v) > 1 else 0.0
        lines.append(f"| {name} | {len(v)} | {sum(v) / len(v):.2f} us | {v[len(v) // 2]:.2f} us "
                     f"| {v[0]:.2f} us | {v[-1]:.2f} us | {sd:.2f} us |")
    counters = {}
    for p in ("fetch", "write", "occ", "lds", "l2"):
        counters.update(counter_means(os.path.join(root, p)))
    lines += ["", "| kernel | counter | mean per dispatch |", "|---|---|---|"]
    for (k, c), v in sorted(counters.items()):
        lines.append(f"| {k} | {c} | {v:,.0f} |")
    stall = counter_means(os.path.join(root, "stall"))
    breakdowns = {k: stall_breakdown(stall, k) for k in sorted({k for k, _ in stall})}
    breakdowns = {k: b for k, b in breakdowns.items() if b}
    if breakdowns:
        lines += ["", "Wave-cycle breakdown (fractions of SQ_WAVE_CYCLES; a wave can wait and",
                  "issue in the same cycle, so the parts need not sum to 1):", "",
                  "| kernel | " + " | ".join(label for label, _ in STALL_PARTS) + " | top 3 |",
                  "|---|" + "---|" * (len(STALL_PARTS) + 1)]
        for k, b in breakdowns.items():
            frac = dict(b)
            top = ", ".join(f"{label} {f:.0%}" for label, f in b[:3])
            lines.append(f"| {k} | " + " | ".join(
                f"{frac[label]:.3f}" if label in frac else "-" for label, _ in STALL_PARTS)
                + f" | {top} |")
    occ = occupancy_rows(os.path.join(root, "trace"))
    if occ:
        lines += ["", "Occupancy (waves per SIMD each resource allows; the smallest limits):", "",
                  "| kernel | VGPRs+AGPRs | LDS bytes | waves/workgroup | by VGPRs | by LDS | "
                  "by grid | limiter |", "|---|---|---|---|---|---|---|---|"]
        for k, r in sorted(occ.items()):
            limits, limiter = occupancy(r)
            wg = int(r["Workgroup_Size_X"]) * int(r["Workgroup_Size_Y"]) * int(r["Workgroup_Size_Z"])
            vg = int(r.get("VGPR_Count") or 0) + int(r.get("Accum_VGPR_Count") or 0)
            lines.append(f"| {k} | {vg} | {r.get('LDS_Block_Size', '')} | {-(-wg // 64)} | "
                         f"{limits.get('VGPRs', '-')} | {limits.get('LDS', '-')} | "
                         f"{limits['grid']:.2f} | {limiter} |")
    cal = calibration(root)
    coal = coalescing(counters, cal)
    if coal:
        lines += ["", "Coalescing (the counterpart of the reference extractor's sectors per request "
                  "and L2 bytes, analysis/ncu/extract.py:127-133): HBM bytes fetched (FETCH_SIZE, "
                  "calibrated) per wave-level vector-memory read instruction "
                  "(SQ_INSTS_VMEM_RD), next to the L2 hit rate. A wave's 16-byte-per-lane load "
                  "moves 1024 B when fully coalesced.", "",
                  "| kernel | HBM bytes fetched | VMEM read instructions | bytes per read "
                  "instruction | L2 hit |", "|---|---|---|---|---|"]
        for k, fetched, insts, per, hit in coal:
            lines.append(f"| {k} | {fetched:,.0f} | {insts:,.0f} | {per:,.0f} | "
                         + (f"{hit:.1%}" if hit is not None else "-") + " |")
    traffic = None
    if cal and dur:
        dominant = max(dur, key=lambda k: sum(dur[k]))
        fetch = counters.get((dominant, "FETCH_SIZE"))
        write = counters.get((dominant, "WRITE_SIZE"))
        if fetch is not None and write is not None:
            traffic = (round(fetch * cal[0]), round(write * cal[1]))
            lines += ["", f"Calibration: FETCH_SIZE x {cal[0]:.1f} B, WRITE_SIZE x {cal[1]:.1f} B "
                      f"per unit (copy of {COPY_BYTES} B).",
                      f"Dominant kernel {dominant}: fetch {traffic[0]:,} B, write {traffic[1]:,} B "
                      "per dispatch."]
    return "\n".join(lines), traffic


def traffic_line(root, config, traffic):
    """The profiles/traffic.txt line for this run: config, kernel label and
    split label as bench.py records them, then the calibrated bytes."""
    out = glob.glob(os.path.join(root, "trace.log"))
    split = None
    for f in out:
        for line in open(f):
            if line.startswith("{") and '"metric"' in line:
                cfg = json.loads(line)["config"]
                split = cfg.get("num_splits", cfg.get("launch"))
    kernel = "mla" if config.startswith("mla") else "v2"
    return f"{config} {kernel} {split} {traffic[0]} {traffic[1]}" if split is not None else None


def bench_line(root):
    """The JSON line bench.py printed in the trace pass, or None."""
    for f in glob.glob(os.path.join(root, "trace.log")):
        for line in open(f):
            if line.startswith("{") and '"metric"' in line:
                return json.loads(line)
    return None


def build_command(bench_args):
    """The build.py command that makes the variant library a --lib bench
    argument names (its defines from the library's provenance record), or
    None for the shipped library."""
    parts = bench_args.split()
    if "--lib" not in parts:
        return None
    lib = parts[parts.index("--lib") + 1]
    sys.path.insert(0, os.path.join(os.path.dirname(HERE), "python"))
    import provenance

    defines = provenance.library_defines(os.path.join(REPO_ROOT, lib)) or []
    name = os.path.basename(os.path.dirname(lib))
    return " ".join(["python mla-decode-kernels_amd/build.py --variant", name] +
                    [f"--define {d}" for d in defines])


def profile_markdown(root, config, argv, summary, build=None):
    """A complete profiles/*.md: what ran, the command that made it, the
    traced run's bench line, then the summary tables."""
    b = bench_line(root) or {}
    occ = occupancy_rows(os.path.join(root, "trace"))
    dur = kernel_durations(os.path.join(root, "trace"))
    dominant = max(dur, key=lambda k: sum(dur[k])) if dur else "?"
    cfg = b.get("config", {})
    title = f"# {dominant.split('::')[-1].split('<')[0]} -- config {config}: " \
            f"{cfg.get('workload', config).split(': ', 1)[-1]}"
    out = [title, ""]
    desc = [f"MI355X ({b.get('gcn_arch', 'gfx950')}, {b.get('cus', '?')} CUs), one GPU."]
    launch = cfg.get("num_splits", cfg.get("launch"))
    if launch is not None:
        what = cfg.get("kernel", "MLA decode")
        how = f"at {launch} split{'s' if launch != 1 else ''}" if isinstance(launch, int) \
            else f"({launch})"
        desc.append(f"Launch: {what} {how}.")
    lib = b.get("provenance", {}).get("library_defines")
    if lib:
        desc.append(f"Library: a profiling build with {', '.join(lib)}.")
    r = occ.get(dominant)
    if r:
        g = [int(r[f"Grid_Size_{a}"]) for a in "XYZ"]
        w = [int(r[f"Workgroup_Size_{a}"]) for a in "XYZ"]
        threads = w[0] * w[1] * w[2]
        wgs = (g[0] // w[0]) * (g[1] // w[1]) * (g[2] // w[2])
        desc.append(f"Dominant kernel {dominant}: {wgs} workgroups of {threads} threads "
                    f"({wgs * -(-threads // 64)} waves).")
    if "kv_bytes" in b:
        desc.append(f"Algorithmic bytes per launch: {b['kv_bytes']:,} (K + V rows, 512 B per "
                    "(token, kv-head)).")
    elif "bytes" in b:
        desc.append(f"Algorithmic bytes per step: {b['bytes']:,.0f} and FLOPs {b['flops']:,.0f} "
                    "(FlashMLA's accounting).")
    desc.append("The copy passes calibrate FETCH_SIZE and WRITE_SIZE on a plain 1 GiB copy "
                "(`bench.py --copy-probe 1024`).")
    out += [" ".join(desc), "",
            "Command (from the repository root; one rocprofv3 process per pass, run from /tmp "
            "with TMPDIR=/tmp, the program after `--` being `python bench.py ...`; the script's "
            "docstring lists each pass's counters; `<dir>` is any absolute output directory):",
            "", "    " + (build + " && " if build else "") +
            "python mla-decode-kernels_amd/bench/profile_config.py " + " ".join(
                a if " " not in a else f'"{a}"' for a in argv), ""]
    if b:
        rl = b.get("roofline", {})
        prov = b.get("provenance", {})
        out += [f"Bench line of the traced run: median step {b.get('value')} us, dominant kernel "
                f"average {rl.get('avg_kernel_us')} us over its back-to-back launches (HIP events "
                f"on the launch stream), roofline.frac {rl.get('frac')}; sources "
                f"{prov.get('source_sha16')} ({prov.get('path')} path, "
                f"mla-decode-kernels_amd/python/provenance.py).", ""]
    out += ["## Kernel trace, counters, wave-cycle breakdown, occupancy and coalescing "
            "(per dispatch)", "", summary, ""]
    return "\n".join(out)


TRAFFIC_FILE = os.path.join(REPO_ROOT, "profiles", "traffic.txt")


def update_traffic(path, line):
    """Replace the line with the same config, kernel and split label (the
    first three fields), or append it; comment lines are kept."""
    key = line.split()[:3]
    kept, replaced = [], False
    for ln in open(path).read().splitlines():
        if not ln.startswith("#") and ln.split()[:3] == key:
            if not replaced:
                kept.append(line)
                replaced = True
            continue
        kept.append(ln)
    if not replaced:
        kept.append(line)
    with open(path, "w") as f:
        f.write("\n".join(kept) + "\n")


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--config", default="c2",
                    choices=["c1", "c2", "c3", "c4", "c5"] + MLA_CONFIGS)
    ap.add_argument("--out-dir", default=None)
    ap.add_argument("--passes", default=",".join(PASSES))
    ap.add_argument("--timeout", type=int, default=300, help="seconds per pass")
    ap.add_argument("--summarize", default=None, help="only summarize an existing output dir")
    ap.add_argument("--bench-args", default="",
                    help="extra bench.py arguments for every pass but the copies")
    ap.add_argument("--profile-md", default=None,
                    help="also write the complete profile file (header, command, tables) here")
    ap.add_argument("--update-traffic", action="store_true",
                    help="replace (or add) this run's line in profiles/traffic.txt, which "
                         "bench.py reads for roofline.traffic")
    args = ap.parse_args(argv)
    root = args.summarize or args.out_dir
    if root is None:
        ap.error("give --out-dir (run and summarize) or --summarize <dir>")
    if not args.summarize:
        run_passes(args.config, root, [p for p in args.passes.split(",") if p], args.timeout,
                   args.bench_args.split())
    text, traffic = summarize(root)
    with open(os.path.join(root, "summary.md"), "w") as f:
        f.write(text + "\n")
    print(text)
    if args.profile_md:
        shown = ["--config", args.config, "--out-dir", "<dir>"]
        if args.passes != ",".join(PASSES):
            shown += ["--passes", args.passes]
        if args.bench_args:
            shown += ["--bench-args", args.bench_args]
        shown += ["--profile-md", os.path.relpath(os.path.abspath(args.profile_md), REPO_ROOT)]
        with open(args.profile_md, "w") as f:
            f.write(profile_markdown(root, args.config, shown, text, build_command(args.bench_args)))
        print(f"wrote {args.profile_md}")
    if traffic:
        line = traffic_line(root, args.config, traffic)
        if line:
            print("traffic line:", line)
            if args.update_traffic:
                update_traffic(TRAFFIC_FILE, line)
                print(f"updated {os.path.relpath(TRAFFIC_FILE, REPO_ROOT)}")


if __name__ == "__main__":
    main()
