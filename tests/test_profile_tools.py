"""The rocprofv3 pass runner and its summary (CPU: command shapes and the
reduction of synthetic rocprofv3 CSV output)."""

import csv
import json
import os
import re

import pytest

import profile_config as pc

# Per-pass hardware limits of one rocprofv3 --pmc run on this GPU, in counter
# units (FETCH_SIZE takes 3 TCC units, WRITE_SIZE 2).
TCC_UNITS = {"FETCH_SIZE": 3, "WRITE_SIZE": 2, "TCC_HIT_sum": 1, "TCC_MISS_sum": 1}


@pytest.mark.parametrize("name", list(pc.PASSES))
def test_pass_commands(name):
    cmd = pc.command(name, "c5", "/tmp/x")
    # The program follows "--" directly (no env/sh/launcher in between).
    i = cmd.index("--")
    assert cmd[i + 1].endswith("python") or "python" in os.path.basename(cmd[i + 1])
    assert cmd[i + 2].endswith("bench.py")
    opts = pc.PASSES[name]
    if "--pmc" in opts:
        assert not {"--kernel-trace", "--sys-trace", "-s", "--runtime-trace", "-r"} & set(opts)
        counters = opts[opts.index("--pmc") + 1:]
        assert sum(c.startswith("SQ_") for c in counters) <= 8
        assert sum(TCC_UNITS.get(c, 0) for c in counters if c in TCC_UNITS) <= 4
        assert sum(c.startswith("GRBM_") for c in counters) <= 2
    if name.startswith("copy_"):
        assert cmd[-2:] == ["--copy-probe", "1024"]
    else:
        assert cmd[cmd.index("--config") + 1] == "c5"


def write_csv(path, rows):
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)


def test_summarize(tmp_path):
    root = str(tmp_path)
    scan = "void gqa::gqa_decode_balanced_kernel<4, 4, 2, true>(gqa::ScanArgs, gqa::BalancedArgs)"
    merge = "void gqa::gqa_decode_balanced_merge_kernel<4, 4>(gqa::ScanArgs, gqa::BalancedArgs)"
    trace = [dict(Kernel_Name=scan, Start_Timestamp=0, End_Timestamp=1_000_000),
             dict(Kernel_Name=scan, Start_Timestamp=0, End_Timestamp=1_200_000),
             dict(Kernel_Name=scan, Start_Timestamp=0, End_Timestamp=1_100_000),
             dict(Kernel_Name=merge, Start_Timestamp=0, End_Timestamp=5_000),
             dict(Kernel_Name="void other_kernel()", Start_Timestamp=0, End_Timestamp=9)]
    write_csv(os.path.join(root, "trace", "x", "run_kernel_trace.csv"), trace)

    def counters(pass_name, kernel, name, values):
        write_csv(os.path.join(root, pass_name, "x", "run_counter_collection.csv"),
                  [dict(Kernel_Name=kernel, Counter_Name=name, Counter_Value=v) for v in values])

    neg = "void at::native::vectorized_elementwise_kernel<4, at::native::neg_kernel_cuda(...)"
    counters("copy_fetch", neg, "FETCH_SIZE", [524288, 524288])   # KiB-like units
    counters("copy_write", neg, "WRITE_SIZE", [1048576])
    counters("fetch", scan, "FETCH_SIZE", [1000, 1002])
    counters("write", scan, "WRITE_SIZE", [8])
    counters("lds", scan, "SQ_INSTS_VMEM_RD", [2002])
    write_csv(os.path.join(root, "l2", "x", "run_counter_collection.csv"),
              [dict(Kernel_Name=scan, Counter_Name="TCC_HIT_sum", Counter_Value=1),
               dict(Kernel_Name=scan, Counter_Name="TCC_MISS_sum", Counter_Value=3)])
    with open(os.path.join(root, "trace.log"), "w") as f:
        f.write("progress line\n" + json.dumps({"metric": "m", "config": {"num_splits": "balanced"}})
                + "\n")

    text, traffic = pc.summarize(root)
    assert "gqa::gqa_decode_balanced_kernel<4, 4, 2, true> | 3 | 1100.00 us | 1100.00 us" in text
    assert "other_kernel" not in text
    # 2^30 bytes per 524288 units = 2048 B per FETCH unit, 1024 per WRITE unit.
    assert traffic == (1001 * 2048, 8 * 1024)
    assert pc.traffic_line(root, "c5", traffic) == f"c5 v2 balanced {1001 * 2048} {8 * 1024}"
    # Coalescing: 1001 x 2048 bytes over 2002 read instructions = 1024 B each;
    # L2 hit 1 of 4.
    assert "| gqa::gqa_decode_balanced_kernel<4, 4, 2, true> | 2,050,048 | 2,002 | 1,024 | 25.0% |" \
        in text
    md = pc.profile_markdown(root, "c5", ["--config", "c5", "--out-dir", "<dir>"], text)
    assert md.startswith("# gqa_decode_balanced_kernel -- config c5")
    assert "profile_config.py --config c5 --out-dir <dir>" in md and text in md


def test_short_name_drops_signature_and_anonymous_namespace():
    assert pc.short_name("void gqa::(anonymous namespace)::gqa_decode_mfma_kernel<8, 16, true, "
                         "true>(gqa::ScanArgs)") == "gqa::gqa_decode_mfma_kernel<8, 16, true, true>"
    assert pc.short_name("gqa::gqa_decode_merge_kernel(float const*, int)") == \
        "gqa::gqa_decode_merge_kernel"


def test_stall_breakdown_and_occupancy(tmp_path):
    root = str(tmp_path)
    k = "void gqa::(anonymous namespace)::gqa_decode_scan_kernel<4, 4, true>(gqa::ScanArgs)"
    res = dict(LDS_Block_Size=90112, VGPR_Count=96, Accum_VGPR_Count=0, SGPR_Count=48,
               Workgroup_Size_X=256, Workgroup_Size_Y=1, Workgroup_Size_Z=1,
               Grid_Size_X=2048, Grid_Size_Y=32, Grid_Size_Z=1)
    write_csv(os.path.join(root, "trace", "x", "run_kernel_trace.csv"),
              [dict(Kernel_Name=k, Start_Timestamp=0, End_Timestamp=160_000, **res)])
    vals = {"SQ_WAVE_CYCLES": 1000, "SQ_WAIT_ANY": 700, "SQ_WAIT_INST_ANY": 100,
            "SQ_ACTIVE_INST_VALU": 300, "SQ_ACTIVE_INST_VMEM": 50, "SQ_ACTIVE_INST_LDS": 20,
            "SQ_ACTIVE_INST_SCA": 10, "SQ_ACTIVE_INST_MISC": 5}
    write_csv(os.path.join(root, "stall", "x", "run_counter_collection.csv"),
              [dict(Kernel_Name=k, Counter_Name=c, Counter_Value=v) for c, v in vals.items()])
    b = pc.stall_breakdown(pc.counter_means(os.path.join(root, "stall")),
                           pc.short_name(k))
    assert [label for label, _ in b[:3]] == ["dependency wait", "VALU/MFMA issue", "issue wait"]
    assert dict(b)["dependency wait"] == pytest.approx(0.7)
    # 96 VGPRs -> 5 waves per SIMD; 88 KiB of LDS -> 1 workgroup of 4 waves per CU
    # -> 1 wave per SIMD; 2048 x 32 threads = 1024 waves = 1 per SIMD on 256 CUs.
    limits, limiter = pc.occupancy(res)
    assert limits["VGPRs"] == 5 and limits["LDS"] == 1 and limits["grid"] == 1
    assert limiter in ("LDS", "grid")
    text, _ = pc.summarize(root)
    assert "dependency wait 70%" in text and "| 96 | 90112 | 4 |" in text


@pytest.mark.gpu
def test_issue_probe_rates(gpu, capsys):
    # The committed issue-rate probes behind the MLA kernel's wave layout run
    # and give physically sensible rates: eight MFMA chains near the dense
    # bf16 peak, and two waves per SIMD hiding FMAs under the matrix unit
    # better than one wave does.
    import issue_probe

    assert issue_probe.main(["--iters", "4000"]) == 0
    out = capsys.readouterr().out
    rows = {}
    for ln in out.splitlines():
        cells = [c.strip() for c in ln.strip("|").split("|")]
        if len(cells) == 7 and cells[0] in ("mfma", "valu", "mfma + valu"):
            rows[(cells[0], int(cells[1]), int(cells[2]), int(cells[3]))] = float(cells[4])
    assert ("mfma", 1, 8, 0) in rows and ("mfma + valu", 2, 4, 8) in rows
    ns_per_mfma = rows[("mfma", 1, 8, 0)] / 8
    assert 5.0 < ns_per_mfma < 20.0  # 16 cycles at 0.8..3.2 GHz
    one = rows[("mfma + valu", 1, 4, 8)] / rows[("mfma", 1, 4, 0)]
    two = rows[("mfma + valu", 2, 4, 8)] / rows[("mfma", 2, 4, 0)]
    assert two < one
    assert "ds_read_b128" in out


@pytest.mark.gpu
def test_lane_swap_semantics(gpu):
    # The row exchanges the decode kernels' cross-row reductions are built on
    # (gqa_device.hpp: xor16_pair, xor32_pair): with x = lane id as both
    # operands, v_permlane16_swap_b32 leaves lane l holding x[l] in one result
    # and x[l ^ 16] in the other (odd 16-lane rows of the first operand swapped
    # with even rows of the second), v_permlane32_swap_b32 x[l] and x[l ^ 32]
    # (upper half of the first operand swapped with the lower half of the
    # second).
    import ctypes

    import numpy as np

    import issue_probe

    lib = ctypes.CDLL(issue_probe.LIB)
    out = np.zeros(256, dtype=np.uint32)
    assert lib.issue_probe_lane_swaps(out.ctypes.data_as(ctypes.c_void_p)) == 0
    x = np.arange(64, dtype=np.uint32)
    odd_row, upper = (x // 16) % 2 == 1, x >= 32
    np.testing.assert_array_equal(out[:64], np.where(odd_row, x - 16, x))
    np.testing.assert_array_equal(out[64:128], np.where(odd_row, x, x + 16))
    np.testing.assert_array_equal(out[128:192], np.where(upper, x - 32, x))
    np.testing.assert_array_equal(out[192:], np.where(upper, x, x + 32))
    for a, b, k in ((out[:64], out[64:128], 16), (out[128:192], out[192:], 32)):
        assert (np.minimum(a, b) == np.minimum(x, x ^ k)).all()
        assert (np.maximum(a, b) == np.maximum(x, x ^ k)).all()


@pytest.mark.gpu
def test_mla_phase_table(gpu, capsys):
    # The phase table of the MLA_PHASE_TIMING build (build.py makes it with
    # every build, from the tree's sources) accounts for the whole kernel:
    # phases within a few percent of the wave's cycles.
    import provenance

    lib = os.path.join(os.path.dirname(pc.HERE), "_build", "phase", "libgqa_decode_hip.so")
    assert os.path.exists(lib), f"{lib} missing: run mla-decode-kernels_amd/build.py"
    assert provenance.library_hash("mla", lib) == provenance.source_hash("mla"), (
        "the phase-timing build is stale: rebuild with mla-decode-kernels_amd/build.py")
    import mla_phases

    # The process has already loaded the in-tree library (capi.lib(), the
    # torch extension): the tool must still run the profiling build.
    import capi

    capi.lib()
    assert mla_phases.main(["--config", "mla_4k", "--steps", "3"]) == 0
    out = capsys.readouterr().out
    assert "Cycles per full interval and wave" in out
    m = re.search(r"Split kernel per wave: (\d+) cycles at (\d+) MHz", out)
    assert m, out
    cycles, mhz = int(m.group(1)), int(m.group(2))
    assert cycles > 10000 and 500 < mhz < 3000, (cycles, mhz)
    rows = {}
    for ln in out.splitlines():
        cells = [c.strip() for c in ln.strip("|").split("|")]
        if cells[0] in ("PV-first 0-3", "QK-first 4-7"):
            rows[cells[0]] = [int(c) for c in cells[1:]]
    for name, vals in rows.items():
        # copies .. barrier add up to the total; an interval of 32 tokens x 128
        # rows holds 2176 MFMA cycles per SIMD, so it cannot be shorter.
        assert sum(vals[:-1]) == pytest.approx(vals[-1], abs=6), (name, vals)
        assert 2176 < vals[-1] < 20000, (name, vals)
    assert len(rows) == 2
    # The full intervals are most of a wave's time at mla_4k.
    share = re.search(r"\| (\d+) \((\d+)%\) \|", out)
    assert share and 50 <= int(share.group(2)) <= 100, out


@pytest.mark.gpu
def test_stream_probe_patterns(gpu, capsys):
    # bench.py --stream-probe: every pattern reads config 2's 1 GiB of K and V
    # at a physical rate; the timed patterns record every workgroup's end (in
    # order: first <= median <= last, the last within the launch); the dynamic
    # pattern leaves its claim counters at zero, and the paged reads cover
    # both pools exactly once (stream_probe checks both).
    import torch

    import bench
    import cases

    assert bench.stream_probe(torch, cases, gpu) == 0
    line = [ln for ln in capsys.readouterr().out.splitlines() if ln.startswith('{"stream_probe"')]
    res = json.loads(line[-1])["results"]
    for key in ("head_strided_nt", "head_strided_plain", "whole_slot_nt", "linear_nt",
                "linear_64wg_4w", "linear_64wg_16w", "linear_128wg_4w", "linear_128wg_16w",
                "head_strided_c3_1split", "head_strided_c3_2split", "paged_identity",
                "paged_shuffled", "timed_head_strided", "dynamic_512", "dynamic_1024"):
        assert 1.0 < res[key]["tbps"] < 8.0, (key, res[key])
    for key in ("timed_head_strided", "dynamic_512", "dynamic_1024"):
        e = res[key]["wg_end_us"]
        assert 0 < e["min"] <= e["p10"] <= e["p50"] <= e["p90"] <= e["max"], (key, e)
        assert e["max"] < 2 * res[key]["median_us"], (key, e, res[key]["median_us"])


def test_update_traffic_replaces_or_appends(tmp_path):
    path = tmp_path / "traffic.txt"
    path.write_text("# header\nc2 v2 1 10 20\nc3 v2 4 30 40\n")
    pc.update_traffic(str(path), "c2 v2 1 11 21")
    pc.update_traffic(str(path), "c5 v2 balanced 50 60")
    assert path.read_text() == "# header\nc2 v2 1 11 21\nc3 v2 4 30 40\nc5 v2 balanced 50 60\n"


@pytest.mark.parametrize("args,want", [
    (("v2", 4, False, 8, 1, 4, 512, 256), "gqa_decode_mfma_kernel"),   # config 1: short splits, idle CUs
    (("v1", 4, False, 8, 1, 1, 512, 256), "gqa_decode_mfma_kernel"),
    (("v2", 4, False, 8, 32, 1, 8192, 256), "gqa_decode_scan_kernel"),  # config 2
    (("v2", 4, False, 8, 32, 32, 8192, 256), "gqa_decode_split_range_kernel"),
    (("v2", 4, False, 8, 8, 4, 32768, 256), "gqa_decode_scan_kernel"),  # config 3
    (("v2", 4, False, 8, 8, 1, 32768, 256), "gqa_decode_scan_kernel"),  # idle CUs, long splits
    (("v2", 4, False, 8, 8, 16, 32768, 256), "gqa_decode_split_range_kernel"),
    (("v2", 8, False, 8, 32, 8, 32768, 256), "gqa_decode_mfma_kernel"),
    (("v2", 8, True, 8, 32, 1, 32768, 256), "gqa_decode_balanced_mfma_kernel"),
    (("v2", 4, True, 16, 32, 1, 32768, 256), "gqa_decode_balanced_kernel"),
    (("v0", 4, False, 8, 1, 1, 512, 256), "gqa_decode_v0_kernel")])
def test_bench_kernel_name(args, want):
    # bench.py's roofline label follows the launchers' routing (the split-range
    # layout from 4 * max(1, CUs // (B * Hkv)) splits; the matrix-core scan on
    # grids of fewer workgroups than CUs with splits of at most 1024 tokens).
    import bench

    assert bench.kernel_name(*args) == want
