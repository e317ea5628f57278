"""Code-generation checks of the MLA decode kernels (CPU: hipcc cross-compiles
csrc/mla_decode.hip for gfx950 to assembly).

The kernels' speed rests on properties of the generated code that a compiler
change or an innocent-looking edit can silently break, so they are checked here:
  - no scratch (spill) access inside the tile loops: with two waves per SIMD a
    wave has 256 registers, of which the 128 PV accumulators and the 72 Q^T
    registers take 200, and a spill reload waits for every HBM->LDS copy in
    flight;
  - no compiler-inserted vmcnt wait inside the tile loops (the copies are
    awaited only by the kernel's own s_waitcnt before each barrier);
  - no compiler use of M0: the copies set M0 in inline assembly, and M0 is a
    register the compiler reserves (it would not restore it).
"""

import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "mla-decode-kernels_amd", "csrc", "mla_decode.hip")
HIPCC = "/opt/rocm/bin/hipcc"

pytestmark = pytest.mark.skipif(not shutil.which(HIPCC), reason="hipcc not available")


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    out = tmp_path_factory.mktemp("mla_asm") / "mla_decode.s"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang",
                    "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S",
                    f"-I{os.path.join(ROOT, 'include')}",
                    f"-I{os.path.join(ROOT, 'mla-decode-kernels_amd', 'csrc')}", SRC, "-o",
                    str(out)], check=True, capture_output=True)
    return out.read_text()


def kernel_body(asm, mangled):
    """The kernel's code: from its label to its end-of-function label (a
    kernel may end its waves early, so it can hold several s_endpgm)."""
    start = asm.index(f"\n{mangled}:")
    return asm[start:asm.index("\n.Lfunc_end", start)]


BLOCK_START = re.compile(r"(\.LBB\w+:|; %bb\.\d+:)")


def tile_loops(body):
    """(text of each loop that issues MFMAs itself, with the loops nested in
    it: the blocks the compiler's loop annotations place there, in layout
    order). A header block is annotated "Loop Header" (and "Parent Loop X" when
    nested), any other block "in Loop: Header=X"."""
    blocks = []
    for ln in body.split("\n"):
        if BLOCK_START.match(ln) or not blocks:
            blocks.append([])
        blocks[-1].append(ln)
    parent, inner = {}, []
    for blk in blocks:
        lab = re.match(r"\.L(BB\w+):", blk[0])
        notes = []
        for ln in blk:  # the leading comment lines
            s = ln.strip()
            if s and not s.startswith(";") and not BLOCK_START.match(s):
                break
            notes.append(s)
        note = " ".join(notes)
        if "Loop Header" in note and lab:
            me = lab.group(1)
            up = re.search(r"Parent Loop (BB\w+)", note)
            parent[me] = up.group(1) if up else None
            inner.append(me)
        else:
            m = re.search(r"in Loop: Header=(BB\w+)", note)
            inner.append(m.group(1) if m else None)
    def chain(h):
        out = []
        while h:
            out.append(h)
            h = parent.get(h)
        return out
    direct = {h for blk, h in zip(blocks, inner) if h and any("v_mfma" in ln for ln in blk)}
    # The tile loops: loops issuing MFMAs with no MFMA-issuing loop inside
    # (a balanced kernel's loop over pieces holds the tile loops).
    tiles = [h for h in direct if not any(h in chain(d)[1:] for d in direct)]
    return ["\n".join("\n".join(blk) for blk, h in zip(blocks, inner) if h and top in chain(h))
            for top in sorted(tiles)]


KERNELS = ["_ZN3mla17mla_decode_kernelILb1EEEvNS_7MlaArgsE",
           "_ZN3mla17mla_decode_kernelILb0EEEvNS_7MlaArgsE",
           "_ZN3mla26mla_decode_balanced_kernelILb1EEEvNS_7MlaArgsE",
           "_ZN3mla26mla_decode_balanced_kernelILb0EEEvNS_7MlaArgsE"]


@pytest.mark.parametrize("mangled", KERNELS)
def test_tile_loops_clean(asm, mangled):
    loops = tile_loops(kernel_body(asm, mangled))
    assert loops, "no tile loop found"
    for text in loops:
        code = [ln for ln in text.split("\n") if ln.strip() and not ln.strip().startswith(";")]
        assert not [ln for ln in code if "scratch_" in ln], "spill access inside a tile loop"
        # Waits the compiler inserted (outside the ;;#ASMSTART blocks) must
        # not name vmcnt.
        own = re.sub(r";;#ASMSTART.*?(;;#ASMEND|\Z)", "", text, flags=re.S)
        assert "vmcnt" not in own, "compiler vmcnt wait inside a tile loop"
        # One interval: QK^T of 16 rows x 32 tokens (36) and PV of 128 rows x
        # 64 dims (32).
        assert text.count("v_mfma_f32_16x16x32_bf16") == 68


@pytest.mark.parametrize("mangled", KERNELS)
def test_m0_only_in_inline_asm(asm, mangled):
    outside = re.sub(r";;#ASMSTART.*?;;#ASMEND", "", kernel_body(asm, mangled), flags=re.S)
    assert not re.search(r"\bm0\b", outside)


def is_vote_address(line):
    """The restart votes sit in the second P buffer, after the tile ring (4 tiles
    of 36 KiB): LDS byte offsets of 128 KiB and up, added to the wave's index
    as an immediate."""
    m = re.search(r"s_add\w*\s+s\d+,\s*s\d+,\s*0x([0-9a-f]+)", line)
    return bool(m) and int(m.group(1), 16) >= 0x20000


@pytest.mark.parametrize("mangled", KERNELS)
def test_restart_ballot_sees_every_lane(asm, mangled):
    # The second-pass vote is a ballot over the wave's `beaten` flags, stored
    # by lane 0. The ballot (a v_cmp into vcc) must be evaluated before the
    # lane-0 branch narrows the exec mask: inside it, it would see lane 0 only.
    lines = kernel_body(asm, mangled).split("\n")
    stores = [i for i, ln in enumerate(lines)
              if "ds_write_b32" in ln and any(is_vote_address(p) for p in lines[max(0, i - 8):i])]
    assert stores, "restart vote store not found"
    for i in stores:
        # The branch narrows exec with s_and_saveexec or by writing exec.
        k = max(k for k in range(i) if re.search(r"s_and_saveexec|s_(mov|and)_b64 exec,", lines[k]))
        between = [ln for ln in lines[k:i] if re.search(r"\bv_cmp", ln)]
        assert not between, f"ballot evaluated under the lane-0 exec mask: {between}"
        assert any(re.search(r"v_cmp\w*\s+vcc", ln) for ln in lines[max(0, k - 30):k]), \
            "ballot not found before the lane-0 branch"


@pytest.fixture(scope="module")
def llvm_ir(tmp_path_factory):
    out = tmp_path_factory.mktemp("mla_ir") / "mla_decode.ll"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang",
                    "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S",
                    "-emit-llvm", f"-I{os.path.join(ROOT, 'include')}",
                    f"-I{os.path.join(ROOT, 'mla-decode-kernels_amd', 'csrc')}", SRC, "-o",
                    str(out)], check=True, capture_output=True)
    return out.read_text()


def test_row_max_uses_both_swap_results(llvm_ir):
    # row_max: each permlane16/32 swap returns the lane's own value and its
    # partner's; the max must use both. A front-end lowering of bit casts of
    # vector elements once read element 0 for both, so the optimised IR kept
    # only result 0 and the "max" was one lane's value.
    calls = re.findall(r"(%[\w.]+) = (?:tail )?call \{ i32, i32 \} @llvm\.amdgcn\.permlane(?:16|32)\.swap",
                       llvm_ir)
    assert calls, "no permlane swap found"
    for v in calls:
        assert re.search(rf"extractvalue \{{ i32, i32 \}} {re.escape(v)}, 1\b", llvm_ir), \
            f"second result of {v} unused"


def test_phase_timing_build_keeps_tile_loops_clean(tmp_path):
    # The profiling build (MLA_PHASE_TIMING, read by bench/mla_phases.py) adds
    # shader-clock stamps to the tile loops; its numbers describe the shipped
    # kernel only if the stamps add no spills there.
    out = tmp_path / "mla_phase.s"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang",
                    "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S",
                    "-DMLA_PHASE_TIMING=1", f"-I{os.path.join(ROOT, 'include')}",
                    f"-I{os.path.join(ROOT, 'mla-decode-kernels_amd', 'csrc')}", SRC, "-o",
                    str(out)], check=True, capture_output=True)
    text = out.read_text()
    assert "mla_phase_cycles" in text
    for mangled in KERNELS:
        loops = tile_loops(kernel_body(text, mangled))
        assert loops
        for loop in loops:
            assert "s_memtime" in loop
            code = [ln for ln in loop.split("\n") if ln.strip() and not ln.strip().startswith(";")]
            assert not [ln for ln in code if "scratch_" in ln]
