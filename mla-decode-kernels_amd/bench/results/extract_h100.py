"""Extract the reference's published H100 matrix medians for side-by-side
reports (run once, in a checkout where the reference is present).

Source: bench/results/matrix_20260824_213534/matrix_summary.csv of the
reference (H100 SXM, CUDA 12.8; its README.md:240-279 tables are generated
from the same files). Kept: per cell, the median time and % of the H100's
3.35 TB/s SoL of FlashInfer 0.6.17, v1 and v2 (best over num_splits
{1,4,8,16,32,64}, with the winning count).

usage: python extract_h100.py <reference checkout> [out.csv]
"""

import csv
import os
import sys

SUMMARY = os.path.join("bench", "results", "matrix_20260824_213534", "matrix_summary.csv")
FIELDS = ["headtype", "S", "B", "block", "kernel", "best_splits", "median_ms", "pct_of_sol"]


def main():
    ref = sys.argv[1]
    out = sys.argv[2] if len(sys.argv) > 2 else os.path.join(os.path.dirname(
        os.path.abspath(__file__)), "h100_reference_matrix.csv")
    with open(os.path.join(ref, SUMMARY)) as f:
        rows = [r for r in csv.DictReader(f) if r["kernel"] in ("flashinfer", "v1", "v2")]
    rows.sort(key=lambda r: (r["headtype"], int(r["S"]), int(r["B"]), int(r["block"]), r["kernel"]))
    with open(out, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=FIELDS, lineterminator="\n")
        w.writeheader()
        for r in rows:
            w.writerow({k: r[k] for k in FIELDS})
    print(f"wrote {out} ({len(rows)} rows)")


if __name__ == "__main__":
    main()
