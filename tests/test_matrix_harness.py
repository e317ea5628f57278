"""The benchmark-matrix harness on the GPU: one small cell driven through
run_matrix.py's command line into a temporary directory, as the reference's
bench/run_matrix.py:140-175 runs its cells (resumable per-cell JSON, summary
CSV rebuilt from the cell files).

Checked: every spot check of the cell passed (v1, v2's automatic choice, the
token-balanced launch and the SDPA baseline, each against an fp32 reference on
the first requests; a failed spot check raises, so a cell file exists only if
all passed); the cell record carries the reference's keys
(bench/run_matrix.py:121-128 of the reference) with consistent values -- the
KV bytes and SoL of the cell, pct_of_sol = sol_ms / median_ms * 100 for every
variant, the best split count the argmin of the sweep; v0 is timed because
S <= 2048 and B <= 8; the record is stamped with the library's provenance,
matching the tree's sources; the CSV holds the reference's columns
(bench/run_matrix.py:117-124) and one row per variant; and a second run
resumes (keeps the existing cell)."""

import csv
import json
import os

import pytest

import cases
import run_matrix

pytestmark = pytest.mark.gpu

CELL = (32, 8, 512, 8, 16)
NAME = run_matrix.cell_name(*CELL)
REFERENCE_KEYS = {"Hq", "Hkv", "S", "B", "block", "warmup", "runs", "kv_bytes", "sol_ms",
                  "spot_check", "results"}
REFERENCE_COLUMNS = ["headtype", "S", "B", "block", "kernel", "best_splits", "median_ms",
                     "pct_of_sol"]


def test_matrix_cell_end_to_end(gpu, tmp_path, capsys):
    argv = ["--out-dir", str(tmp_path), "--only", NAME, "--warmup", "2", "--runs", "5"]
    print(f"matrix cell {NAME}", flush=True)
    run_matrix.main(argv)
    path = tmp_path / f"{NAME}.json"
    cell = json.loads(path.read_text())

    assert REFERENCE_KEYS <= set(cell)
    Hq, Hkv, S, B, bs = CELL
    assert (cell["Hq"], cell["Hkv"], cell["S"], cell["B"], cell["block"]) == CELL
    assert (cell["warmup"], cell["runs"]) == (2, 5)
    assert cell["provenance"]["path"] == "gqa"
    assert cell["provenance"]["library_matches_sources"], cell["provenance"]
    assert cell["kv_bytes"] == S * B * Hkv * 128 * 2 * 2
    assert cell["sol_ms"] == pytest.approx(cell["kv_bytes"] / cases.HBM_PEAK_BYTES_PER_S * 1e3)

    assert set(cell["spot_check"]) == {"v1", "v2_auto", "balanced", "sdpa"}
    for label, verdict in cell["spot_check"].items():
        assert verdict.startswith("passed"), (label, verdict)
        assert float(verdict.split("max-abs ")[1].rstrip(")")) <= 2e-2

    res = cell["results"]
    assert set(res) == {"sdpa", "v1", "v2", "v2_auto", "balanced", "v0"}
    for label, r in res.items():
        assert r["median_ms"] > 0
        assert r["pct_of_sol"] == pytest.approx(cell["sol_ms"] / r["median_ms"] * 100), label
    by = {int(k): v for k, v in res["v2"]["by_splits"].items()}
    assert sorted(by) == run_matrix.SPLITS_LIST
    assert res["v2"]["best_splits"] == min(by, key=by.get)
    assert res["v2"]["median_ms"] == by[res["v2"]["best_splits"]]
    choice = res["v2_auto"]["choice"]
    assert choice == "balanced" or (isinstance(choice, int) and choice >= 1)

    with open(tmp_path / "matrix_summary.csv", newline="") as f:
        reader = csv.DictReader(f)
        rows = list(reader)
    assert reader.fieldnames[:len(REFERENCE_COLUMNS)] == REFERENCE_COLUMNS
    assert "ratio_vs_sdpa" in reader.fieldnames
    assert sorted(r["kernel"] for r in rows) == sorted(res)
    for r in rows:
        assert r["headtype"] == f"{Hq}x{Hkv}" and int(r["S"]) == S and int(r["B"]) == B
        assert float(r["ratio_vs_sdpa"]) == pytest.approx(
            res["sdpa"]["median_ms"] / res[r["kernel"]]["median_ms"])
    assert next(r for r in rows if r["kernel"] == "v2")["best_splits"] == \
        str(res["v2"]["best_splits"])

    # A second run over the same directory resumes: the cell is not rerun.
    mtime = os.path.getmtime(path)
    capsys.readouterr()
    run_matrix.main(argv)
    assert "1 of 1 cells already recorded" in capsys.readouterr().out
    assert os.path.getmtime(path) == mtime
