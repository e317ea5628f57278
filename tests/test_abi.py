"""CPU tests of the drop-in boundary: the C ABI library and the torch operator
layer, without launching anything (this container has no GPU).

Covers: every function include/gqa_decode.h declares is exported; the
workspace-size and split-count entry points; argument rejection before any
launch (hipErrorInvalidValue); the torch op's input checks and messages
(python/gqa_decode_ext.cpp:16-62,102-103 of the reference).
"""

import ctypes
import math

import pytest
import torch

import capi

INVALID = capi.HIP_ERROR_INVALID_VALUE


def test_library_exports_every_declared_function():
    declared = capi.declared_functions()
    assert declared == sorted([
        "gqa_decode_v0_launch", "gqa_decode_v1_launch", "gqa_decode_v2_launch",
        "gqa_decode_v2_partial_launch", "gqa_decode_v2_merge_launch",
        "gqa_decode_v2_workspace_bytes", "gqa_decode_v2_fused_launch",
        "gqa_decode_v2_fused_workspace_bytes", "gqa_decode_v2_fused_reset",
        "gqa_decode_pick_num_splits",
        "gqa_decode_balanced_launch", "gqa_decode_balanced_workspace_bytes",
        "gqa_decode_balanced_partial_launch", "gqa_decode_balanced_merge_launch",
        "gqa_decode_balanced_launch_noalloc", "gqa_decode_prefer_balanced",
    ])
    lib = capi.lib()
    for name in declared:
        assert hasattr(lib, name), f"{name} not exported"


def test_library_exports_nothing_else():
    import subprocess

    out = subprocess.run(["nm", "-D", "--defined-only", capi.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    names = {ln.split()[-1] for ln in out.splitlines() if ln.strip()}
    assert {n for n in names if n.startswith("gqa")} == set(capi.declared_functions())


@pytest.mark.parametrize("B,Hq,ns", [(32, 32, 8), (1, 32, 1), (128, 64, 512), (3, 5, 7)])
def test_workspace_bytes(B, Hq, ns):
    assert capi.workspace_bytes(B, Hq, ns) == B * Hq * ns * (128 + 2) * 4


@pytest.mark.parametrize("args", [(0, 32, 8), (32, 0, 8), (32, 32, 0), (-1, 32, 8)])
def test_workspace_bytes_invalid(args):
    assert capi.workspace_bytes(*args) == 0


WAVES_PER_HEAD = 4     # waves sharing a kv-head
MIN_SPLIT_TOKENS = 2 * 16 * WAVES_PER_HEAD  # two 16-token tiles per wave
MAX_CHUNK = 8192
MAX_SPLITS = 32
SLOT_CHUNK = 4096      # longest split of the matrix-core slot-group layout
SLOT_MIN_CHUNK = 1024  # its shortest
SLOT_WAVES_PER_CU = 8  # its residency: one workgroup of Hkv waves, two per SIMD


def waves_per_split(B, Hq, Hkv):
    G = Hq // Hkv
    per_wave = 16 if G >= 5 else (1 if G <= 1 else 2 if G <= 2 else 4)
    return B * Hkv * -(-G // per_wave) * WAVES_PER_HEAD


def target_waves(Hq, Hkv, s_max, cus):
    mfma = Hq // Hkv >= 5
    return cus * (8 if mfma and s_max >= 8192 else 4)


def slot_shape(Hq, Hkv):
    """Groups the matrix-core scan's slot-group layout serves."""
    return 5 <= Hq // Hkv <= 16 and Hkv in (4, 8)


def slot_eligible(B, Hkv, ns, cus):
    """Its grid gives at least 3/4 of the CUs their 8 resident waves."""
    return B * ns * Hkv * 4 >= 3 * SLOT_WAVES_PER_CU * cus


@pytest.mark.parametrize("Hq,Hkv", [(32, 8), (64, 8), (32, 4)])
@pytest.mark.parametrize("B,max_blocks,bs", [(1, 1, 16), (1, 8, 16), (1, 32, 16), (1, 512, 64),
                                             (3, 512, 16), (8, 512, 64), (32, 512, 16),
                                             (32, 512, 64), (64, 512, 16), (100, 512, 16),
                                             (128, 2048, 16), (4096, 64, 16), (2, 100000, 16)])
def test_pick_num_splits_properties(B, max_blocks, bs, Hq, Hkv):
    cus = 256
    s_max = max_blocks * bs
    ns = capi.pick_num_splits(B, Hq, Hkv, bs, max_blocks, cus)
    if slot_shape(Hq, Hkv):
        # Slot-group layout: one workgroup per CU (rounded down), no split
        # longer than SLOT_CHUNK, none shorter than SLOT_MIN_CHUNK, at most 32.
        cap = min(MAX_SPLITS, max(1, s_max // SLOT_MIN_CHUNK))
        fill = SLOT_WAVES_PER_CU * cus // (B * Hkv)
        want = min(cap, max(fill, -(-s_max // SLOT_CHUNK), 1))
        if slot_eligible(B, Hkv, want, cus):
            assert ns == want
            return
    per = waves_per_split(B, Hq, Hkv)
    target = target_waves(Hq, Hkv, s_max, cus)
    cap = min(MAX_SPLITS, max(1, s_max // MIN_SPLIT_TOKENS))
    assert 1 <= ns <= cap
    length = -(-s_max // MAX_CHUNK)
    if ns < cap:
        # No split longer than MAX_CHUNK ...
        assert -(-s_max // ns) <= MAX_CHUNK
        # ... and the fill bound is maximal: one more split would overfill
        # the round of resident waves.
        assert (ns + 1) * per > target
    if ns > 1 and ns > length:
        # Splits beyond the length bound only fill the round, never overfill it.
        assert ns * per <= target


def test_pick_num_splits_headline_shapes():
    # BASELINE configs 1..5 on 256 CUs: the representative shape fills the
    # chip without splitting; fewer, longer requests split more.
    assert capi.pick_num_splits(1, 32, 8, 16, 32, 256) == 4
    assert capi.pick_num_splits(32, 32, 8, 16, 512, 256) == 1
    assert capi.pick_num_splits(8, 32, 8, 64, 512, 256) == 4
    assert capi.pick_num_splits(32, 64, 8, 64, 512, 256) == 8  # slot-group layout
    assert capi.pick_num_splits(128, 32, 8, 16, 2048, 256) == 4
    prev = 0
    for B in (128, 32, 8, 1):
        cur = capi.pick_num_splits(B, 32, 8, 64, 512, 256)
        assert cur >= prev
        prev = cur


@pytest.mark.parametrize("args", [(0, 32, 8, 16, 512, 256), (32, 30, 8, 16, 512, 256),
                                  (32, 32, 0, 16, 512, 256), (32, 32, 8, 0, 512, 256),
                                  (32, 32, 8, 16, 0, 256)])
def test_pick_num_splits_invalid(args):
    assert capi.pick_num_splits(*args) == 0


FAKE = 0x1000  # never dereferenced: every call below is rejected before a launch


def launch_args(**over):
    a = dict(q=FAKE, k=FAKE, v=FAKE, bt=FAKE, sl=FAKE, out=FAKE, B=2, Hq=32, Hkv=8, bs=16,
             max_blocks=4, scale=0.088)
    a.update(over)
    return [a[k] for k in ("q", "k", "v", "bt", "sl", "out", "B", "Hq", "Hkv", "bs",
                           "max_blocks", "scale")]


BAD = [dict(Hq=30), dict(Hkv=0), dict(Hq=0), dict(bs=0), dict(max_blocks=0), dict(B=-1),
       dict(B=70000), dict(q=None), dict(k=None), dict(v=None), dict(bt=None), dict(sl=None),
       dict(out=None), dict(bs=1 << 20, Hkv=64)]


@pytest.mark.parametrize("over", BAD)
def test_launchers_reject_bad_arguments(over):
    args = launch_args(**over)
    assert capi.v0_launch(*args, None) == INVALID
    assert capi.v1_launch(*args, None) == INVALID
    assert capi.v2_launch(*args, 8, FAKE, FAKE, FAKE, None) == INVALID


@pytest.mark.parametrize("ns", [0, -1, 513])
def test_v2_rejects_num_splits(ns):
    assert capi.v2_launch(*launch_args(), ns, FAKE, FAKE, FAKE, None) == INVALID
    assert capi.v2_partial_launch(*launch_args()[:5], *launch_args()[6:], ns, FAKE, FAKE, FAKE,
                                  None) == INVALID
    assert capi.v2_merge_launch(FAKE, FAKE, FAKE, FAKE, 2, 32, ns, None) == INVALID


@pytest.mark.parametrize("which", [0, 1, 2])
def test_v2_rejects_missing_workspace(which):
    ws = [FAKE, FAKE, FAKE]
    ws[which] = None
    assert capi.v2_launch(*launch_args(), 8, *ws, None) == INVALID
    assert capi.v2_merge_launch(*ws, FAKE, 2, 32, 8, None) == INVALID


@pytest.mark.parametrize("B,Hq,ns", [(32, 32, 8), (1, 32, 1), (128, 64, 512), (3, 5, 7),
                                     (1, 1, 1)])
def test_fused_workspace_bytes(B, Hq, ns):
    # Arrival counters (4 bytes per (request, q-head), padded to 256 bytes)
    # first, then the v2 workspace.
    counters = (4 * B * Hq + 255) // 256 * 256
    assert capi.fused_workspace_bytes(B, Hq, ns) == counters + capi.workspace_bytes(B, Hq, ns)


@pytest.mark.parametrize("args", [(0, 32, 8), (32, 0, 8), (32, 32, 0), (-1, 32, 8)])
def test_fused_workspace_bytes_invalid(args):
    assert capi.fused_workspace_bytes(*args) == 0


def fused_args(ns=8, ws=FAKE, ws_bytes=None, **over):
    a = launch_args(**over)
    if ws_bytes is None:
        ws_bytes = capi.fused_workspace_bytes(max(a[6], 1), max(a[7], 1), max(ns, 1))
    return a + [ns, ws, ws_bytes, None]


@pytest.mark.parametrize("over", BAD)
def test_fused_rejects_bad_arguments(over):
    assert capi.v2_fused_launch(*fused_args(**over)) == INVALID


def test_fused_rejects_bad_workspace():
    # Split counts out of range, a missing, misaligned or short workspace.
    for ns in (0, -1, 513):
        assert capi.v2_fused_launch(*fused_args(ns=ns, ws_bytes=1 << 30)) == INVALID
    assert capi.v2_fused_launch(*fused_args(ws=None)) == INVALID
    assert capi.v2_fused_launch(*fused_args(ws=FAKE + 4)) == INVALID
    need = capi.fused_workspace_bytes(2, 32, 8)
    assert capi.v2_fused_launch(*fused_args(ws_bytes=need - 1)) == INVALID
    # The reset checks the same workspace rules before launching its fill.
    for args in [(None, need, 2, 32, 8), (FAKE + 4, need, 2, 32, 8), (FAKE, need - 1, 2, 32, 8),
                 (FAKE, need, 2, 32, 0), (FAKE, need, -1, 32, 8), (FAKE, need, 2, 0, 8)]:
        assert capi.v2_fused_reset(*args, None) == INVALID
    # Empty batches launch nothing.
    assert capi.v2_fused_reset(None, 0, 0, 32, 8, None) == capi.HIP_SUCCESS
    assert capi.v2_fused_launch(*fused_args(B=0, q=None, k=None, v=None, bt=None, sl=None,
                                            out=None, ws=None)) == capi.HIP_SUCCESS


@pytest.mark.parametrize("Hq,Hkv,nwg,gh", [(32, 8, 256, 4), (8, 8, 256, 1), (16, 8, 7, 2),
                                          (24, 8, 256, 4), (4, 1, 1, 4), (64, 16, 256, 4),
                                          (6, 2, 9, 4), (32, 16, 3, 2), (16, 16, 256, 1),
                                          # groups of 5-16 (matrix-core scan): all Hq heads
                                          (64, 8, 256, 64), (40, 8, 3, 40), (128, 8, 256, 128),
                                          (32, 4, 256, 32), (64, 4, 5, 64)])
def test_balanced_workspace_bytes(Hq, Hkv, nwg, gh):
    # Two partial states (first and last piece) per workgroup, 132 floats per
    # head of a slot, then a 32-byte share record per workgroup at a 16-byte
    # boundary. A slot holds all Hq q-heads with 4 or 8 kv-heads (matrix-core
    # scan), else one kv-head's q-heads rounded to 1, 2 or 4 (VALU scan).
    if Hkv in (4, 8):
        gh = Hq
    states = (nwg * 2 * gh * 132 * 4 + 15) // 16 * 16
    assert capi.balanced_workspace_bytes(32, Hq, Hkv, nwg) == states + nwg * 32


@pytest.mark.parametrize("args", [(0, 32, 8, 256), (32, 136, 8, 256), (32, 30, 8, 256),
                                  (32, 32, 0, 256), (32, 48, 6, 256), (32, 128, 16, 256),
                                  (32, 16, 2, 256)])
def test_balanced_workspace_bytes_invalid(args):
    assert capi.balanced_workspace_bytes(*args) == 0


def balanced_args(ws_bytes=1 << 20, nwg=256, **over):
    return launch_args(**over) + [nwg, FAKE, ws_bytes, None]


@pytest.mark.parametrize("over", BAD)
def test_balanced_rejects_bad_arguments(over):
    assert capi.balanced_launch(*balanced_args(**over)) == INVALID


def test_balanced_rejects_unsupported_shapes():
    # Groups above 16 q-heads, groups of 5+ over other than 4 or 8 kv-heads,
    # batches beyond the LDS prefix table, workspace missing or too small for
    # the workgroup count.
    assert capi.balanced_launch(*balanced_args(Hq=136)) == INVALID
    assert capi.balanced_launch(*balanced_args(Hq=96, Hkv=12)) == INVALID
    assert capi.balanced_launch(*balanced_args(Hq=64, Hkv=8, ws_bytes=1 << 20)) == INVALID
    assert capi.balanced_launch(*balanced_args(B=20480)) == INVALID
    args = balanced_args()
    args[-3] = None
    assert capi.balanced_launch(*args) == INVALID
    need = capi.balanced_workspace_bytes(2, 32, 8, 256)
    assert capi.balanced_launch(*balanced_args(ws_bytes=need - 1)) == INVALID


@pytest.mark.parametrize("fn", ["balanced_partial_launch", "balanced_merge_launch"])
@pytest.mark.parametrize("over", BAD + [dict(Hq=136), dict(Hq=96, Hkv=12), dict(B=20480)])
def test_balanced_parts_reject_bad_arguments(fn, over):
    assert getattr(capi, fn)(*balanced_args(**over)) == INVALID


def test_prefer_balanced_headline_shapes():
    # BASELINE configs 1..5 on 256 CUs: balanced for the ragged config (5) and
    # the 8-head groups (4, whose lengths the host cannot tell from ragged
    # ones); the split path where the split grid is exactly one wave per SIMD
    # (2, 3) and for tiny batches (1).
    shapes = [(1, 32, 16, 32), (32, 32, 16, 512), (8, 32, 64, 512), (32, 64, 64, 512),
              (128, 32, 16, 2048)]
    assert [capi.prefer_balanced(B, Hq, 8, bs, mb, 256) for B, Hq, bs, mb in shapes] == \
        [0, 0, 0, 1, 1]


@pytest.mark.parametrize("B,Hq,bs,mb", [(1, 32, 16, 2048), (8, 32, 16, 512), (32, 32, 64, 512),
                                        (128, 32, 16, 2048), (256, 32, 16, 2048), (1, 32, 16, 64),
                                        (4, 16, 16, 4096), (2, 64, 16, 4096), (128, 32, 16, 512),
                                        (64, 32, 16, 512), (600, 32, 16, 1024), (3, 24, 16, 2048),
                                        (1, 32, 16, 512), (128, 32, 16, 511), (512, 32, 16, 256),
                                        # groups of 5-16 (matrix-core scan)
                                        (32, 64, 64, 512), (8, 64, 16, 2048), (8, 64, 16, 512),
                                        (7, 64, 64, 2048), (16, 64, 16, 512), (16, 64, 16, 511),
                                        (128, 64, 16, 128), (4, 128, 64, 512), (64, 40, 16, 512)])
@pytest.mark.parametrize("Hkv", [8, 4, 16])
def test_prefer_balanced_rule(B, Hq, bs, mb, Hkv):
    # The documented rule, clause by clause. Hq is given for 8 kv-heads; the
    # same group runs over 4 (matrix-core scan for every group) and 16 (VALU
    # scan for groups of at most 4, no balanced launch above).
    G, cus = Hq // 8, 256
    Hq = G * Hkv
    s_max = mb * bs
    ns = capi.pick_num_splits(B, Hq, Hkv, bs, mb, cus)
    kv_bytes = B * s_max * Hkv * 512
    mfma_batch = B >= 8 and kv_bytes >= 512 << 20
    if G >= 5:
        want = Hkv in (4, 8) and G <= 16 and mfma_batch
    else:
        want = (s_max >= 6144 and kv_bytes >= 32 << 20 and B * Hkv <= 16 * cus
                and not (B * Hkv * 4 * ns == 4 * cus and ns <= 8))
        if Hkv in (4, 8):
            want = want and B >= 8
    assert capi.prefer_balanced(B, Hq, Hkv, bs, mb, cus) == int(want)


def test_prefer_balanced_single_request_small_group():
    # 32Q/8KV, one request of 8192 or 32768 tokens: the matrix-core balanced
    # scan would cut it into a piece per CU (measured 67.5 vs 21.0 us and 81.7
    # vs 34.8 us against the split launch), so the split launch runs.
    assert capi.prefer_balanced(1, 32, 8, 16, 512, 256) == 0
    assert capi.prefer_balanced(1, 32, 8, 64, 512, 256) == 0
    # 128 requests of 8192 tokens keep the balanced launch (641 vs 667 us).
    assert capi.prefer_balanced(128, 32, 8, 16, 512, 256) == 1


def test_prefer_balanced_invalid():
    assert capi.prefer_balanced(0, 32, 8, 16, 512, 256) == 0
    assert capi.prefer_balanced(8, 30, 8, 16, 512, 256) == 0
    assert capi.prefer_balanced(20480, 32, 8, 16, 16, 256) == 0
    # Groups of 5+ over other than 4 or 8 kv-heads, and groups above 16.
    assert capi.prefer_balanced(64, 96, 12, 16, 2048, 256) == 0
    assert capi.prefer_balanced(64, 136, 8, 16, 2048, 256) == 0


def test_empty_batch_is_a_no_op():
    args = launch_args(B=0, q=None, k=None, v=None, bt=None, sl=None, out=None)
    assert capi.v0_launch(*args, None) == capi.HIP_SUCCESS
    assert capi.v1_launch(*args, None) == capi.HIP_SUCCESS
    assert capi.v2_launch(*args, 8, None, None, None, None) == capi.HIP_SUCCESS
    assert capi.balanced_launch(*args, 256, None, 0, None) == capi.HIP_SUCCESS


# ----------------------------------------------------------- torch operator


@pytest.fixture(scope="module")
def binding():
    import binding as b
    return b


def cpu_case(B=2, Hq=32, Hkv=8, bs=16, nb=8, mb=4):
    q = torch.zeros(B, Hq, 128, dtype=torch.bfloat16)
    k = torch.zeros(nb, bs, Hkv, 128, dtype=torch.bfloat16)
    bt = torch.zeros(B, mb, dtype=torch.int32)
    sl = torch.ones(B, dtype=torch.int32)
    return q, k, k.clone(), bt, sl


def test_binding_exports(binding):
    assert set(binding.KERNELS) == {"v0", "v1", "v2"}
    assert binding.KERNELS["v2"] is binding.gqa_decode_v2
    assert binding.EXTENSION_PATH.startswith(capi._PKG_DIR)
    assert binding.num_splits_heuristic(32, 32, 8, 16, 512, 256) == \
        capi.pick_num_splits(32, 32, 8, 16, 512, 256)


@pytest.mark.parametrize("B,Hq,bs,mb", [(1, 32, 16, 32), (8, 64, 64, 8), (1, 32, 16, 33),
                                        (8, 32, 64, 512), (128, 32, 16, 512), (32, 64, 64, 512),
                                        (2, 32, 1, 512), (2, 32, 1, 513)])
def test_op_automatic_choice(binding, B, Hq, bs, mb):
    # gqa_decode_v2(num_splits=0): the balanced launch (0) where
    # gqa_decode_prefer_balanced says so, else one split for block tables of
    # at most 512 tokens, else the C ABI heuristic's count.
    cus = 256
    if capi.prefer_balanced(B, Hq, 8, bs, mb, cus):
        want = 0
    elif mb * bs <= 512:
        want = 1
    else:
        want = capi.pick_num_splits(B, Hq, 8, bs, mb, cus)
    assert binding.automatic_choice(B, Hq, 8, bs, mb, cus) == want


@pytest.mark.parametrize("kernel", ["v0", "v1", "v2"])
def test_op_rejects_host_tensors(binding, kernel):
    with pytest.raises(RuntimeError, match="q must be a CUDA tensor"):
        binding.KERNELS[kernel](*cpu_case(), 0.088)


def test_op_check_order_and_messages(binding):
    # Checks run in the reference's order, so the first failing one names it.
    q, k, v, bt, sl = cpu_case()
    with pytest.raises(RuntimeError, match="q must be a CUDA tensor"):
        binding.gqa_decode_v2(q.float(), k, v, bt, sl, 0.088, num_splits=4)
    with pytest.raises(TypeError):
        binding.gqa_decode_v2(q, k, v, bt, sl, 0.088, num_splits="x")


# ------------------------------------------------------------ MLA decode ABI


def test_mla_exports():
    declared = capi.declared_mla_functions()
    assert declared == ["mla_decode_balanced_launch", "mla_decode_balanced_workspace_bytes",
                        "mla_decode_combine_launch", "mla_decode_launch",
                        "mla_decode_pick_num_splits", "mla_decode_splitkv_launch",
                        "mla_decode_workspace_bytes"]
    import subprocess

    out = subprocess.run(["nm", "-D", "--defined-only", capi.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    names = {ln.split()[-1] for ln in out.splitlines() if ln.strip()}
    assert {n for n in names if n.startswith("mla")} == set(declared)


@pytest.mark.parametrize("B,s_q,h_q,ns", [(128, 1, 128, 2), (1, 2, 16, 64), (3, 1, 5, 7)])
def test_mla_workspace_bytes(B, s_q, h_q, ns):
    assert capi.mla_workspace_bytes(B, s_q, h_q, ns) == B * s_q * h_q * ns * (512 + 2) * 4
    assert capi.mla_workspace_bytes(B, s_q, h_q, 1) == 0


@pytest.mark.parametrize("B,s_q,h_q,nwg", [(128, 1, 128, 256), (1, 2, 128, 256), (7, 1, 16, 100),
                                           (3, 2, 200, 64)])
def test_mla_balanced_workspace_bytes(B, s_q, h_q, nwg):
    R = s_q * h_q
    n = max(1, nwg // ((R + 127) // 128))
    states = 2 * n * R
    a16 = lambda x: (x + 15) // 16 * 16  # noqa: E731
    want = a16(states * 514 * 4) + (B + 2) * 8
    assert capi.mla_balanced_workspace_bytes(B, s_q, h_q, nwg) == want
    assert capi.mla_balanced_workspace_bytes(0, s_q, h_q, nwg) == 0


def test_mla_pick_num_splits():
    # One workgroup per CU: 128 requests of 128 rows -> 2 splits on 256 CUs;
    # one long request -> capped by 256-token splits and the 128 maximum.
    assert capi.mla_pick_num_splits(128, 1, 128, 64, 512, 256) == 2
    assert capi.mla_pick_num_splits(1, 1, 128, 64, 512, 256) == 128
    assert capi.mla_pick_num_splits(1, 1, 128, 64, 4, 256) == 1
    assert capi.mla_pick_num_splits(64, 1, 256, 64, 512, 256) == 2  # two row groups
    assert capi.mla_pick_num_splits(0, 1, 128, 64, 512, 256) == 0


def mla_args(**over):
    a = dict(q=FAKE, kv=FAKE, bt=FAKE, sl=FAKE, out=FAKE, lse=FAKE, B=2, s_q=1, h_q=16, bs=64,
             mb=4, scale=0.04, causal=0, ns=1, ws=None, wsb=0)
    a.update(over)
    return [a[k] for k in ("q", "kv", "bt", "sl", "out", "lse", "B", "s_q", "h_q", "bs", "mb",
                           "scale", "causal", "ns", "ws", "wsb")] + [None]


@pytest.mark.parametrize("over", [dict(B=-1), dict(B=70000), dict(s_q=0), dict(h_q=0),
                                  dict(bs=0), dict(mb=0), dict(ns=0), dict(ns=129),
                                  dict(q=None), dict(kv=None), dict(bt=None), dict(sl=None),
                                  dict(out=None), dict(ns=4, ws=None, wsb=1 << 20),
                                  dict(ns=4, ws=FAKE + 4, wsb=1 << 20), dict(ns=4, wsb=16,
                                                                             ws=FAKE)])
def test_mla_rejects_bad_arguments(over):
    assert capi.mla_launch(*mla_args(**over)) == INVALID
    assert capi.mla_splitkv_launch(*mla_args(**over)) == INVALID


@pytest.mark.parametrize("over", [dict(B=-1), dict(B=70000), dict(s_q=0), dict(h_q=0),
                                  dict(bs=0), dict(mb=0), dict(q=None), dict(kv=None),
                                  dict(bt=None), dict(sl=None), dict(out=None), dict(ws=None),
                                  dict(ws=FAKE + 4), dict(wsb=16)])
def test_mla_balanced_rejects_bad_arguments(over):
    a = mla_args(**{**dict(ns=256, ws=FAKE, wsb=1 << 30), **over})
    assert capi.mla_balanced_launch(*a) == INVALID


@pytest.mark.parametrize("over", [dict(ns=1), dict(ns=0), dict(ns=129), dict(B=-1),
                                  dict(s_q=0), dict(h_q=0), dict(out=None), dict(ws=None),
                                  dict(ws=FAKE + 4), dict(wsb=16)])
def test_mla_combine_rejects_bad_arguments(over):
    a = dict(ws=FAKE, wsb=1 << 30, out=FAKE, lse=FAKE, B=2, s_q=1, h_q=16, ns=4)
    a.update(over)
    assert capi.mla_combine_launch(*[a[k] for k in ("ws", "wsb", "out", "lse", "B", "s_q", "h_q",
                                                    "ns")], None) == INVALID


def test_mla_empty_batch_is_a_no_op():
    assert capi.mla_launch(*mla_args(B=0, q=None, kv=None, bt=None, sl=None, out=None,
                                     lse=None)) == capi.HIP_SUCCESS
    assert capi.mla_combine_launch(None, 0, None, None, 0, 1, 16, 4, None) == capi.HIP_SUCCESS
    assert capi.mla_balanced_launch(*mla_args(B=0, q=None, kv=None, bt=None, sl=None, out=None,
                                              lse=None, ns=256)) == capi.HIP_SUCCESS
