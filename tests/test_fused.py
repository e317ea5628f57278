"""GPU tests of the single-launch split-KV entry point (gqa_decode_v2_fused_launch).

The fused launch runs the split kernel, and the last workgroup of each merge
group to finish folds the group's states with the merge kernel's arithmetic.
So its output must equal gqa_decode_v2_launch's (partial + merge) bit for bit
at every split count, in every launch layout: the VALU scan, the matrix-core
scan head-strided and in the slot-group layout. Also checked:
- the reference's case grid against the fp32 oracle (atol = rtol = 2e-2,
  NaN-poisoned pools);
- arrival counters left at zero after every launch;
- one workspace reused for a smaller batch, and garbage in the state area;
- bitwise repeatability;
- replays of a captured HIP graph against eager launches, with eager work
  between replays.
"""

import numpy as np
import pytest
import torch

import capi
from cases import make_case
from gpu_util import assert_close, numpy_oracle
from test_gqa_decode import ATOL, CASES, RTOL, SCALE, alloc_ws, ref_case, stream_ptr

pytestmark = pytest.mark.gpu


def shape(case):
    q, k, _, bt, _ = case
    return q.shape[0], q.shape[1], k.shape[2], k.shape[1], bt.shape[1]


def fused_workspace(B, Hq, ns, device, fill=None):
    """A fused-launch workspace for (B, Hq, ns), counters reset."""
    n = capi.fused_workspace_bytes(B, Hq, ns)
    ws = torch.empty((n + 3) // 4, dtype=torch.float32, device=device)
    if fill is not None:
        ws.fill_(fill)
    assert capi.v2_fused_reset(ws.data_ptr(), n, B, Hq, ns, stream_ptr()) == 0
    return ws, n


def counters(ws, B, Hq):
    return ws[:B * Hq].view(torch.int32)


def fused(case, ns, ws, n, out=None):
    q, k, v, bt, sl = case
    B, Hq, Hkv, bs, mb = shape(case)
    out = torch.empty_like(q) if out is None else out
    rc = capi.v2_fused_launch(q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(),
                              sl.data_ptr(), out.data_ptr(), B, Hq, Hkv, bs, mb, SCALE, ns,
                              ws.data_ptr(), n, stream_ptr())
    assert rc == 0
    return out


def two_launch(case, ns):
    """gqa_decode_v2_launch through the C ABI: partial kernel + merge kernel."""
    q, k, v, bt, sl = case
    B, Hq, Hkv, bs, mb = shape(case)
    out = torch.empty_like(q)
    _, acc, m, l = alloc_ws(B, Hq, ns, q.device)
    rc = capi.v2_launch(q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr(),
                        out.data_ptr(), B, Hq, Hkv, bs, mb, SCALE, ns, acc.data_ptr(),
                        m.data_ptr(), l.data_ptr(), stream_ptr())
    assert rc == 0
    return out


def check_fused(case, ns, label, want=None):
    B, Hq = shape(case)[:2]
    ws, n = fused_workspace(B, Hq, ns, case[0].device, fill=float("nan"))
    out = fused(case, ns, ws, n)
    ref2 = two_launch(case, ns)
    torch.cuda.synchronize()
    assert torch.equal(out, ref2), f"{label}: fused != partial + merge bitwise"
    assert not counters(ws, B, Hq).any(), f"{label}: arrival counters not left at zero"
    if want is not None:
        assert_close(out, want, ATOL, RTOL, label)
    return out


@pytest.mark.parametrize("name", list(CASES))
@pytest.mark.parametrize("ns", [2, 3, 8, 32])
def test_fused_reference_grid(gpu, name, ns):
    print(f"fused {name} ns={ns}", flush=True)
    case = ref_case(CASES[name])
    check_fused(case, ns, f"{name}/ns{ns}", want=numpy_oracle(case, SCALE))


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (16, 8), (24, 8), (32, 8), (40, 8), (64, 8),
                                    (128, 8), (256, 8), (32, 1), (4, 2), (48, 4)])
@pytest.mark.parametrize("bs", [7, 16, 64])
def test_fused_groups_and_block_sizes(gpu, Hq, Hkv, bs):
    # Groups of 1-32 (VALU scan up to 4, matrix-core scan from 5, two q-head
    # chunks at 32), block sizes on and off the 16-token tile.
    print(f"fused Hq={Hq} Hkv={Hkv} bs={bs}", flush=True)
    case = ref_case(dict(S_list=[77, 300, 16, 1, 545], Hq=Hq, Hkv=Hkv, bs=bs), seed=Hq + bs)
    check_fused(case, 5, f"Hq{Hq}/Hkv{Hkv}/bs{bs}", want=numpy_oracle(case, SCALE))


@pytest.mark.parametrize("Hq,Hkv", [(64, 8), (40, 8), (32, 4), (128, 8)])
def test_fused_slot_layout(gpu, Hq, Hkv):
    # Enough (request, split) workgroups for the matrix-core slot-group layout:
    # one workgroup per (split, request) and the request as the merge group.
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    B = 24 if Hkv == 8 else 48
    ns = -(-(24 * cus) // (4 * B * Hkv))
    print(f"fused slot Hq={Hq} Hkv={Hkv} B={B} ns={ns}", flush=True)
    S = np.random.default_rng(Hq).integers(1, 700, size=B).tolist()
    S[:3] = [1, 64, 65]
    case = ref_case(dict(S_list=S, Hq=Hq, Hkv=Hkv, bs=16), seed=Hq)
    check_fused(case, ns, f"slot Hq{Hq}/Hkv{Hkv}", want=numpy_oracle(case, SCALE))


def test_fused_one_split_is_single_pass(gpu):
    case = ref_case(CASES["a_base"])
    check_fused(case, 1, "ns1")


def test_fused_workspace_reuse(gpu):
    # One workspace, reset once for the larger batch, serves a smaller batch
    # and a different group next; the counters stay at zero throughout.
    big = ref_case(dict(S_list=[900, 33, 4000, 257, 1, 128], Hq=64, Hkv=8, bs=16), seed=3)
    ws, n = fused_workspace(6, 64, 16, big[0].device, fill=float("nan"))
    for case, ns in [(big, 16), (ref_case(CASES["a_base"], seed=4), 8),
                     (ref_case(dict(S_list=[5000, 70], Hq=16, Hkv=4, bs=64), seed=5), 16),
                     (big, 7)]:
        B, Hq = shape(case)[:2]
        assert capi.fused_workspace_bytes(B, Hq, ns) <= n
        out = fused(case, ns, ws, n)
        want = two_launch(case, ns)
        torch.cuda.synchronize()
        assert torch.equal(out, want)
        assert not counters(ws, 6, 64).any()


def test_fused_bitwise_repeatable(gpu):
    case = ref_case(CASES["a_base"])
    ws, n = fused_workspace(4, 32, 7, case[0].device)
    first = fused(case, 7, ws, n)
    for _ in range(5):
        assert torch.equal(fused(case, 7, ws, n), first)


def test_fused_graph_replay(gpu):
    # The launch captured once and replayed: each replay is checked against an
    # eager launch on the inputs of the moment, with eager work (a new query,
    # the eager launch itself) between replays.
    case = ref_case(dict(S_list=[700, 64, 3000, 1], Hq=32, Hkv=8, bs=16), seed=8)
    q, k, v, bt, sl = case
    ws, n = fused_workspace(4, 32, 8, q.device)
    out = torch.empty_like(q)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fused(case, 8, ws, n, out)  # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fused(case, 8, ws, n, out)
    ws_eager, n_eager = fused_workspace(4, 32, 8, q.device)
    gen = torch.Generator(device="cpu").manual_seed(9)
    for rep in range(5):
        q.copy_((0.5 * torch.randn(q.shape, generator=gen)).to(q.device, torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        want = fused(case, 8, ws_eager, n_eager)
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {rep} differs from the eager launch"
        assert torch.equal(want, two_launch(case, 8))
        assert not counters(ws, 4, 32).any()


def test_fused_config3_full_size(gpu):
    """BASELINE config 3 (B=8, S=32768, block 64) at its automatic split count."""
    from cases import make_config_case

    case = make_config_case("c3", seed=0, device=torch.device("cuda", 0))
    B, Hq, Hkv, bs, mb = shape(case)
    ns = capi.pick_num_splits(B, Hq, Hkv, bs, mb, 0)
    assert ns > 1
    print(f"fused c3 ns={ns}", flush=True)
    check_fused(case, ns, "c3")


def test_fused_stress_random_shapes(gpu):
    """Bounded stress of the arrival protocol: 40 seeded random shapes
    (kv-heads 1-16, groups 1-16, both scans and both matrix-core layouts,
    block sizes on and off the tile, 2-64 splits, up to 48 ragged requests),
    each launched three times back to back on one workspace, every output
    bitwise equal to partial + merge; stops at the first mismatch."""
    rng = np.random.default_rng(2024)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    for i in range(40):
        Hkv = int(rng.choice([1, 2, 4, 8, 16]))
        G = int(rng.integers(1, 17))
        B = int(rng.integers(1, 49))
        bs = int(rng.choice([1, 7, 16, 64]))
        ns = int(rng.integers(2, 65))
        if i % 4 == 0 and Hkv in (4, 8) and G >= 5:
            ns = max(ns, -(-(24 * cus) // (4 * B * Hkv)))  # the slot-group layout's grid
        S = rng.integers(1, 4097, size=B).tolist()
        label = f"stress {i}: Hq={G * Hkv} Hkv={Hkv} B={B} bs={bs} ns={ns}"
        print(label, flush=True)
        case = make_case(S, G * Hkv, Hkv, bs, pool_factor=1.2, seed=i, qkv_std=0.5)
        want = two_launch(case, ns)
        ws, n = fused_workspace(B, G * Hkv, ns, case[0].device, fill=float("nan"))
        outs = [fused(case, ns, ws, n) for _ in range(3)]
        torch.cuda.synchronize()
        for r, out in enumerate(outs):
            assert torch.equal(out, want), f"{label}: launch {r} differs from partial + merge"
        assert not counters(ws, B, G * Hkv).any(), f"{label}: counters not left at zero"
        del case, ws, outs
