"""The results report is generated only from archived files, and refuses to
publish when the archive is inconsistent (the reference's sanity-anchor rule,
analysis/report/make_report.py:177-216)."""

import copy
import importlib

import pytest

make_report = importlib.import_module("make_report")


def test_committed_report_matches_archive(capsys):
    make_report.main(["--check"])
    assert "check OK" in capsys.readouterr().out


def load():
    return make_report.load_cells(), make_report.load_h100(), make_report.load_bench()


def test_anchors_pass_on_archive():
    make_report.sanity(*load())


@pytest.mark.parametrize("corrupt", ["pct", "best", "missing", "spot", "h100"])
def test_anchors_reject_inconsistent_archive(corrupt):
    cells, h100, bench = load()
    cells = copy.deepcopy(cells)
    h100 = copy.deepcopy(h100)
    rep = cells[make_report.REP]["results"]
    if corrupt == "pct":
        rep["v1"]["pct_of_sol"] *= 1.01
    elif corrupt == "best":
        rep["v2"]["best_splits"] = 64 if rep["v2"]["best_splits"] != 64 else 1
    elif corrupt == "missing":
        del cells[make_report.REP]
    elif corrupt == "spot":
        cells[make_report.REP]["spot_check"]["v1"] = "failed"
    elif corrupt == "h100":
        h100[make_report.REP]["v2"]["median_ms"] = "1.2"
    with pytest.raises(SystemExit, match="SANITY ANCHOR FAILED"):
        make_report.sanity(cells, h100, bench)
