"""MI355X results report, generated only from archived result files.

Counterpart of the reference's analysis/report/make_report.py:177-216,596-682:
every number in results/REPORT.md is computed here from committed files --
the 64-cell matrix (run_matrix.py output), the five BASELINE configs'
bench.py lines, and the reference's H100 matrix medians -- and each section
names its source. Before writing, a set of sanity anchors is re-derived from
those files (complete grid, % of SoL consistent with the times, best split
consistent with the sweep, spot checks passed, the H100 extraction matching
the reference's own anchors); any failure aborts without writing.

Every archived record carries the provenance stamp bench.py and
run_matrix.py write (python/provenance.py): the hash of the sources of the
measured path and the hash the library that ran was built from. --check also
fails when an archived record's stamp differs from the tree's current
sources, so archived numbers cannot outlive the kernels they measured.

  python make_report.py            # regenerate results/REPORT.md
  python make_report.py --check    # exit 1 if the report or any archived record is stale
"""

import argparse
import csv
import json
import os
import statistics
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
RESULTS = os.path.join(HERE, "results")
MATRIX_DIR = os.path.join(RESULTS, "matrix_mi355x")
BENCH_LINES = os.path.join(RESULTS, "bench_configs.jsonl")
MLA_LINES = os.path.join(RESULTS, "bench_mla.jsonl")
H100_CSV = os.path.join(RESULTS, "h100_reference_matrix.csv")
REPORT = os.path.join(RESULTS, "REPORT.md")

HEADTYPES = [32, 64]            # Hq; Hkv = 8 throughout
S_LIST = [512, 2048, 8192, 32768]
B_LIST = [1, 8, 32, 128]
BLOCKS = [16, 64]
SPLITS = [1, 4, 8, 16, 32, 64]
REP = (32, 8192, 32, 16)        # (Hq, S, B, block): the representative cell
PEAK = 8.0e12
KV_BYTES_PER_TOKEN_HEAD = 512   # K + V rows, bf16, d = 128


def rel(path):
    return os.path.relpath(path, os.path.dirname(os.path.dirname(HERE)))


# ---------------------------------------------------------------- loading

def load_cells(matrix_dir=MATRIX_DIR):
    cells = {}
    for fname in sorted(os.listdir(matrix_dir)):
        if fname.startswith("cell_") and fname.endswith(".json"):
            with open(os.path.join(matrix_dir, fname)) as f:
                c = json.load(f)
            cells[(c["Hq"], c["S"], c["B"], c["block"])] = c
    return cells


def load_h100(path=H100_CSV):
    out = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            key = (int(r["headtype"].split("x")[0]), int(r["S"]), int(r["B"]), int(r["block"]))
            out.setdefault(key, {})[r["kernel"]] = r
    return out


def load_bench(path=BENCH_LINES):
    with open(path) as f:
        return [json.loads(ln) for ln in f if ln.strip()]


def load_mla(path=MLA_LINES):
    return load_bench(path)


# ---------------------------------------------------------------- provenance

def current_sources():
    sys.path.insert(0, os.path.join(os.path.dirname(HERE), "python"))
    import provenance
    return {kind: provenance.source_hash(kind) for kind in provenance.SOURCES}


def stale_records(cells, bench, mla, sources):
    """Labels of archived records not stamped with the current sources of
    their path (or measured with a library built from other sources)."""
    stale = []

    def test(label, rec, kind):
        p = rec.get("provenance")
        if not p or p.get("path") != kind or p.get("source_sha16") != sources[kind] \
                or not p.get("library_matches_sources") or p.get("library_defines"):
            got = p.get("source_sha16") if p else "no stamp"
            stale.append(f"{label} ({got}; current {kind} sources {sources[kind]})")

    for (hq, s, b, blk), c in sorted(cells.items()):
        test(f"matrix cell {hq}x8 S{s} B{b} bs{blk}", c, "gqa")
    for rec in bench:
        test(f"bench line {rec['config']['workload'][:2]}", rec, "gqa")
    for rec in mla:
        test(f"MLA bench line {rec['config']['workload'].split(':')[0]}", rec, "mla")
    return stale


# ---------------------------------------------------------------- anchors

def check(cond, what):
    if not cond:
        raise SystemExit(f"SANITY ANCHOR FAILED: {what} -- refusing to write the report")


def close(a, b, tol=1e-6):
    return abs(a - b) <= tol * max(abs(a), abs(b), 1e-12)


def sanity(cells, h100, bench):
    check(len(cells) == 64, f"64 matrix cells (found {len(cells)})")
    for (hq, s, b, blk), c in cells.items():
        name = f"{hq}x8 S{s} B{b} bs{blk}"
        check(c["kv_bytes"] == b * s * 8 * KV_BYTES_PER_TOKEN_HEAD, f"{name}: kv_bytes formula")
        check(close(c["sol_ms"], c["kv_bytes"] / PEAK * 1e3), f"{name}: sol_ms at 8 TB/s")
        r = c["results"]
        for k in ("v1", "v2", "v2_auto", c["baseline"]):
            check(k in r, f"{name}: result {k} present")
        check("balanced" in r, f"{name}: balanced launch timed")
        choice = r["v2_auto"]["choice"]
        check(choice == "balanced" or isinstance(choice, int), f"{name}: automatic choice recorded")
        for k, v in r.items():
            check(close(v["pct_of_sol"], c["sol_ms"] / v["median_ms"] * 100),
                  f"{name}: {k} % of SoL = sol / median")
        by = {int(k): v for k, v in r["v2"]["by_splits"].items()}
        check(sorted(by) == SPLITS, f"{name}: v2 swept over {SPLITS}")
        best = min(by, key=by.get)
        check(r["v2"]["best_splits"] == best and close(r["v2"]["median_ms"], by[best]),
              f"{name}: v2 best is the sweep's minimum")
        check(("v0" in r) == (s <= 2048 and b <= 8), f"{name}: v0 timed iff S<=2048 and B<=8")
        check(all(str(v).startswith("passed") for v in c["spot_check"].values()),
              f"{name}: spot checks passed")
    check(len(h100) == 64 and all(set(v) == {"flashinfer", "v1", "v2"} for v in h100.values()),
          "H100 extraction: 64 cells x {flashinfer, v1, v2}")
    rep = h100[REP]
    # The reference's own anchors on its representative cell
    # (analysis/report/make_report.py:183-190 of the reference).
    check(abs(float(rep["v2"]["median_ms"]) - 1.1426) < 5e-4, "H100 rep v2 best 1.1426 ms")
    check(int(rep["v2"]["best_splits"]) == 32, "H100 rep v2 best splits = 32")
    check(abs(float(rep["flashinfer"]["median_ms"]) - 0.3682) < 5e-4, "H100 rep FlashInfer 0.3682 ms")
    check(sorted(b["config"]["workload"][:2] for b in bench) == ["c1", "c2", "c3", "c4", "c5"],
          "bench lines for configs c1..c5")
    for b in bench:
        # bench.py prints pct_of_sol to 2 decimals: allow half a unit of that.
        sol_us = b["kv_bytes"] / PEAK * 1e6
        check(abs(b["pct_of_sol"] - sol_us / b["value"] * 100) <= 0.0051,
              f"{b['config']['workload'][:2]}: pct_of_sol = sol / value")


# ---------------------------------------------------------------- sections

def us(ms):
    return f"{ms * 1e3:.1f}"


def sec_headline(bench, cells, h100):
    lines = ["## BASELINE configs (`bench.py`, one MI355X)", "",
             "| config | splits | median step (us) | % of 8 TB/s SoL | dominant kernel | kernel avg (us) "
             "| kernel GB/s | HBM traffic / KV bytes |",
             "|---|---|---|---|---|---|---|---|"]
    for b in sorted(bench, key=lambda x: x["config"]["workload"]):
        rf = b["roofline"]
        traffic = f"{rf['traffic'] / b['kv_bytes']:.4f}" if rf.get("traffic") else "-"
        lines.append(
            f"| {b['config']['workload']} | {b['config']['num_splits']} | {b['value']:.1f} "
            f"| {b['pct_of_sol']:.1f} | `{rf['kernel']}` | {rf['avg_kernel_us']:.1f} "
            f"| {rf['achieved']:.0f} | {traffic} |")
    c = cells[REP]["results"]
    hr = h100[REP]
    lines += ["", f"Representative matrix cell (32x8, S=8192, B=32, block 16; the reference's "
              f"timing: events around each op call): v1 {us(c['v1']['median_ms'])} us, v2 best "
              f"{us(c['v2']['median_ms'])} us (ns={c['v2']['best_splits']}), automatic choice "
              f"{us(c['v2_auto']['median_ms'])} us ({choice_label(c['v2_auto'])}, "
              f"{c['v2_auto']['pct_of_sol']:.1f} % of SoL). H100 reference: v2 best "
              f"{us(float(hr['v2']['median_ms']))} us "
              f"(ns={hr['v2']['best_splits']}), FlashInfer {us(float(hr['flashinfer']['median_ms']))} us.",
              "", f"Source: {rel(BENCH_LINES)}, {rel(MATRIX_DIR)}, {rel(H100_CSV)}"]
    return lines


def choice_label(r):
    return "bal." if r["choice"] == "balanced" else f"ns={r['choice']}"


def sec_pershape(cells, h100, block):
    lines = [f"## Per shape, block {block} (median us; x = speed-up)", "",
             "auto = v2 with num_splits=0 (bal. = the token-balanced launch, else the split "
             "heuristic's count); % SoL is auto's.", "",
             "| Hq/Hkv | S | B | v1 | v2 best (ns) | balanced | auto (choice) | % SoL | SDPA "
             "| x SDPA | H100 v2 best | H100 FlashInfer | x H100 FlashInfer |",
             "|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
    for hq in HEADTYPES:
        for s in S_LIST:
            for b in B_LIST:
                c = cells[(hq, s, b, block)]
                r = c["results"]
                h = h100[(hq, s, b, block)]
                base = r[c["baseline"]]["median_ms"]
                auto = r["v2_auto"]["median_ms"]
                fi = float(h["flashinfer"]["median_ms"])
                bal = us(r["balanced"]["median_ms"]) if "balanced" in r else "-"
                lines.append(
                    f"| {hq}/8 | {s} | {b} | {us(r['v1']['median_ms'])} | {us(r['v2']['median_ms'])} "
                    f"({r['v2']['best_splits']}) | {bal} | {us(auto)} ({choice_label(r['v2_auto'])}) "
                    f"| {r['v2_auto']['pct_of_sol']:.1f} | {us(base)} | {base / auto:.2f} "
                    f"| {us(float(h['v2']['median_ms']))} | {us(fi)} | {fi / auto:.2f} |")
    lines += ["", f"Source: {rel(MATRIX_DIR)}, {rel(H100_CSV)}"]
    return lines


def best_ms(r):
    """The best time any launch reached on the cell: the split sweep or the
    token-balanced launch."""
    return min(r["v2"]["median_ms"], r.get("balanced", r["v2"])["median_ms"])


def sec_summary(cells):
    heur_pct = [c["results"]["v2_auto"]["pct_of_sol"] for c in cells.values()]
    regret = sorted((c["results"]["v2_auto"]["median_ms"] / best_ms(c["results"]), k)
                    for k, c in cells.items())
    base = [(c["results"][c["baseline"]]["median_ms"] / c["results"]["v2_auto"]["median_ms"], k)
            for k, c in cells.items()]
    nbal = sum(c["results"]["v2_auto"]["choice"] == "balanced" for c in cells.values())
    blk = []
    for (hq, s, b, bs), c in cells.items():
        if bs == 16:
            o = cells[(hq, s, b, 64)]
            for k in ("v1", "v2_auto"):
                t16, t64 = c["results"][k]["median_ms"], o["results"][k]["median_ms"]
                blk.append((abs(t16 - t64) / min(t16, t64) * 100, (hq, s, b), k))
    sat = [c["results"]["v2_auto"]["pct_of_sol"] for (hq, s, b, bs), c in cells.items()
           if c["kv_bytes"] >= 1 << 30]

    def name(k):
        return f"{k[0]}x8 S{k[1]} B{k[2]} bs{k[3]}"

    lines = ["## Summary over the 64 cells", "",
             f"- Automatic choice (balanced in {nbal} cells, else the split heuristic) vs the best "
             f"of the split sweep {{1,4,8,16,32,64}} and the balanced launch: median ratio "
             f"{statistics.median(x for x, _ in regret):.3f}, best {regret[0][0]:.3f} "
             f"({name(regret[0][1])}), worst {regret[-1][0]:.3f} ({name(regret[-1][1])}); "
             f"{sum(x <= 1.01 for x, _ in regret)} of 64 cells within 1 %.",
             f"- Automatic choice, % of 8 TB/s SoL: median {statistics.median(heur_pct):.1f}, max "
             f"{max(heur_pct):.1f}; over the {len(sat)} cells with >= 1 GiB of KV: median "
             f"{statistics.median(sat):.1f}, min {min(sat):.1f}.",
             f"- Speed-up over the SDPA baseline: median {statistics.median(x for x, _ in base):.2f}x, "
             f"min {min(base)[0]:.2f}x ({name(min(base)[1])}), max {max(base)[0]:.2f}x "
             f"({name(max(base)[1])}).",
             f"- Block size 16 vs 64 (v1 and automatic v2, {len(blk)} pairs): median |difference| "
             f"{statistics.median(x for x, _, _ in blk):.2f} %, {sum(x > 2 for x, _, _ in blk)} pairs "
             f"above 2 %.",
             "", f"Source: {rel(MATRIX_DIR)}"]
    return lines


def sec_argbest(cells):
    lines = ["## Best split count of the sweep (block 16; the automatic choice in brackets)", "",
             "| Hq/Hkv | S | " + " | ".join(f"B={b}" for b in B_LIST) + " |",
             "|---|---|" + "---|" * len(B_LIST)]
    for hq in HEADTYPES:
        for s in S_LIST:
            row = []
            for b in B_LIST:
                r = cells[(hq, s, b, 16)]["results"]
                row.append(f"{r['v2']['best_splits']} ({choice_label(r['v2_auto'])})")
            lines.append(f"| {hq}/8 | {s} | " + " | ".join(row) + " |")
    lines += ["", f"Source: {rel(MATRIX_DIR)}"]
    return lines


def sec_mla(mla):
    lines = ["## K2 MLA absorbed decode (`bench.py --config mla_*`, one MI355X)", "",
             "Source: `" + rel(MLA_LINES) + "`. FlashMLA's accounting (its benchmark's "
             "FLOPs and bytes); H100 column: the reference's FlashMLA log on H100 SXM.", "",
             "| row | causal | launch | median (us) | TFLOP/s | GB/s | % of MFMA peak "
             "| % of HBM peak | FlashMLA H100 (us) |",
             "|---|---|---|---|---|---|---|---|---|"]
    for r in mla:
        cfg = r["config"]
        h100 = r.get("flashmla_h100_us")
        lines.append(
            f"| {cfg['workload'].split(':')[0]} | {'yes' if cfg.get('causal') else 'no'} "
            f"| {cfg.get('launch', '')} | {r['value']:.1f} | {r['tflops']:.1f} | {r['gbps']:.1f} "
            f"| {r['roofline']['mfma_frac'] * 100:.1f} | {r['roofline']['hbm_frac'] * 100:.1f} "
            f"| {h100:.1f} |" if h100 else "| - |")
    return lines


def sec_provenance(cells, bench, mla):
    def hashes(recs):
        return sorted({r.get("provenance", {}).get("source_sha16", "none") for r in recs})
    return ["## Provenance", "",
            "Every archived record is stamped with the hash of the sources of its path "
            "(`mla-decode-kernels_amd/python/provenance.py`); `make_report.py --check` fails "
            "when a stamp differs from the tree.", "",
            f"- GQA matrix cells: sources {', '.join(hashes(cells.values()))}",
            f"- GQA bench lines (c1-c5): sources {', '.join(hashes(bench))}",
            f"- MLA bench lines: sources {', '.join(hashes(mla))}"]


def render(cells, h100, bench, mla=()):
    out = ["# MI355X results: GQA paged decode", "",
           "Generated by `mla-decode-kernels_amd/bench/make_report.py` from archived result "
           "files; do not edit by hand. Times are medians in microseconds; % of SoL is KV bytes "
           "/ 8 TB/s over the median. SDPA is torch's AOTriton attention on the same inputs "
           "gathered to contiguous K/V beforehand (its run() timed only). H100 columns are the "
           "reference's published matrix (H100 SXM, 3.35 TB/s).", ""]
    sections = [sec_headline(bench, cells, h100), sec_summary(cells),
                sec_pershape(cells, h100, 16), sec_pershape(cells, h100, 64), sec_argbest(cells)]
    if mla:
        sections.append(sec_mla(mla))
    sections.append(sec_provenance(cells, bench, mla))
    for sec in sections:
        out += sec + [""]
    return "\n".join(out)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--check", action="store_true",
                    help="regenerate in memory; exit 1 if the committed report is stale")
    args = ap.parse_args(argv)
    cells, h100, bench, mla = load_cells(), load_h100(), load_bench(), load_mla()
    sanity(cells, h100, bench)
    text = render(cells, h100, bench, mla)
    if args.check:
        stale = stale_records(cells, bench, mla, current_sources())
        if stale:
            print(f"STALE ARCHIVE: {len(stale)} records were not measured on the current sources:")
            for label in stale[:20]:
                print(f"  {label}")
            sys.exit(1)
        try:
            with open(REPORT) as f:
                same = f.read() == text
        except FileNotFoundError:
            same = False
        if not same:
            print(f"STALE: {rel(REPORT)} does not match the archived data")
            sys.exit(1)
        print("check OK: the report matches the archived data, all stamped with the current "
              "sources")
        return
    with open(REPORT, "w") as f:
        f.write(text)
    print(f"wrote {rel(REPORT)}")


if __name__ == "__main__":
    main()
