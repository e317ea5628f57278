"""GPU tests of v2's split-range layout (gqa_decode_split_range_kernel).

With at least as many splits as the split launch gives each (request,
kv-head) waves -- 4 * max(1, CUs // (B * Hkv)) for groups of up to 4 q-heads
-- every split is scanned by one wave, and each wave walks a contiguous run
of splits with one tile pipeline. The batches here are sized from the
device's CU count so that this layout is the one that runs. Checked:
- every (request, q-head, split) workspace state against the oracle's state
  of the same token range (ragged lengths, splits that are empty, splits
  shorter than a tile, runs of 1 or 2 splits per wave when the split count is
  not a multiple of the wave count), for 16-token blocks and for blocks of 7
  tokens (the per-lane gather path), with NaN in every slot that must not be
  read;
- the output of the whole batch against the oracle;
- states that do not depend on how splits are dealt to waves: the same
  requests in a batch with 1 workgroup per pair and in one with 2 or 4 give
  the same bits;
- the single-launch form equal to partial + merge bit for bit, counters left
  at zero;
- v2 with the in-workgroup merge equal to partial + merge bit for bit, on
  both sides of the LDS stage's capacity (mid-run drains), up to the largest
  split count (512);
- replays of captured HIP graphs of each form equal to the eager launches;
- bitwise repeatability.
"""

import numpy as np
import pytest
import torch

import capi
from binding import gqa_decode_v2
from cases import make_case
from gpu_util import assert_close, host_case, oracle
from oracle import c_oracle
from oracle import reference as ref
from test_gqa_decode import SCALE, alloc_ws, build_segments, stream_ptr
from test_fused import counters, fused, fused_workspace, two_launch

pytestmark = pytest.mark.gpu

# Edge lengths first (shorter than a tile, one tile, a tile and a token, two
# tiles and a token, exact blocks), then longer ones.
EDGE = [1, 15, 16, 17, 33, 64, 100, 257, 1000, 2048, 3001, 4096]


def cus():
    return torch.cuda.get_device_properties(0).multi_processor_count


def groups_per_pair(B, Hkv):
    """Workgroups per (request, kv-head) of the split launch (the launch's
    rule for groups of up to 4 q-heads)."""
    return max(1, cus() // (B * Hkv))


def lengths(B, seed, top=4096):
    rng = np.random.default_rng(seed)
    S = list(rng.integers(1, top + 1, size=B))
    S[:len(EDGE)] = EDGE[:B]
    return [int(s) for s in S]


def partial(case, ns):
    q, k, v, bt, sl = case
    B, Hq, Hkv, bs, mb = q.shape[0], q.shape[1], k.shape[2], k.shape[1], bt.shape[1]
    ws, acc, m, l = alloc_ws(B, Hq, ns, q.device)
    ws.fill_(float("nan"))
    rc = capi.v2_partial_launch(q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(),
                                sl.data_ptr(), B, Hq, Hkv, bs, mb, SCALE, ns, acc.data_ptr(),
                                m.data_ptr(), l.data_ptr(), stream_ptr())
    assert rc == 0
    torch.cuda.synchronize()
    return ws, acc, m, l


def check_states(case, acc, m, l, ns, requests):
    """States of the given requests against the C oracle's partial_state."""
    qh, kh, vh, bth, slh = host_case(case)
    G = qh.shape[1] // kh.shape[2]
    acc_h, m_h, l_h = acc.cpu().numpy(), m.cpu().numpy(), l.cpu().numpy()
    assert np.isfinite(acc_h[requests]).all(), "a state was left unwritten"
    for b in requests:
        S = int(slh[b])
        _, V = ref.gather_kv(kh, vh, bth, S, b)
        for h in range(qh.shape[1]):
            for i, (a, e) in enumerate(build_segments(S, ns)):
                where = f"b={b} S={S} h={h} split={i} [{a},{e})"
                if a == e:
                    assert m_h[b, h, i] == -np.inf and l_h[b, h, i] == 0, where
                    assert not acc_h[b, h, i].any(), where
                    continue
                mw, lw, aw = c_oracle.partial_state(qh[b, h], kh, vh, bth[b], h // G, a, e, SCALE)
                assert m_h[b, h, i] == pytest.approx(mw, abs=1e-5), where
                assert l_h[b, h, i] == pytest.approx(lw, rel=1e-4), where
                # |acc error| <= 1e-4 * sum_t p_t |v_t| <= 1e-4 * l * max|v|
                vmax = float(np.abs(V[a:e, h // G]).max())
                np.testing.assert_allclose(acc_h[b, h, i], aw, rtol=0, atol=1e-4 * lw * vmax,
                                           err_msg=where)


@pytest.mark.parametrize("bs", [16, 7])
@pytest.mark.parametrize("ns", [4, 6, 16, 37])
def test_states_and_output(gpu, bs, ns):
    Hq, Hkv = 8, 2
    B = -(-cus() // Hkv)  # one workgroup per (request, kv-head): 4 waves per pair
    assert groups_per_pair(B, Hkv) == 1
    S = lengths(B, seed=ns * 100 + bs)
    print(f"split-range bs={bs} ns={ns} B={B}", flush=True)
    case = make_case(S, Hq, Hkv, bs, pool_factor=1.25, seed=ns + bs, poison=True)
    ws, acc, m, l = partial(case, ns)
    check_states(case, acc, m, l, ns, list(range(len(EDGE))) + [B - 1])
    out = gqa_decode_v2(*case, SCALE, num_splits=ns)
    torch.cuda.synchronize()
    assert_close(out, oracle(case, SCALE), 2e-2, 2e-2, f"split-range bs={bs} ns={ns}")
    assert torch.equal(gqa_decode_v2(*case, SCALE, num_splits=ns), out)


@pytest.mark.parametrize("G", [1, 2, 3])
def test_small_groups(gpu, G):
    """Groups of 1-3 q-heads (one wave serves the group with zero q rows past
    it): states and output."""
    Hkv = 4
    B = -(-cus() // Hkv)
    S = lengths(B, seed=G)
    case = make_case(S, G * Hkv, Hkv, 16, pool_factor=1.25, seed=G, poison=True)
    ws, acc, m, l = partial(case, 8)
    check_states(case, acc, m, l, 8, list(range(6)))
    out = gqa_decode_v2(*case, SCALE, num_splits=8)
    torch.cuda.synchronize()
    assert_close(out, oracle(case, SCALE), 2e-2, 2e-2, f"split-range G={G}")


@pytest.mark.parametrize("z", [2, 4])
def test_states_independent_of_wave_deal(gpu, z):
    """A split's state is the sequential fold of its tiles, whichever wave
    scans it: the first requests of a batch with one workgroup per pair and
    the same requests alone, with z workgroups per pair, give the same bits
    (the split count is a multiple of 4 * z, so both run this layout)."""
    Hq, Hkv, ns = 8, 2, 32
    B1 = -(-cus() // Hkv)
    B2 = cus() // (Hkv * z)
    assert groups_per_pair(B1, Hkv) == 1 and groups_per_pair(B2, Hkv) == z and ns >= 4 * z
    S = lengths(B1, seed=7)
    big = make_case(S, Hq, Hkv, 16, pool_factor=1.25, seed=3, poison=True)
    q, k, v, bt, sl = big
    small = (q[:B2].contiguous(), k, v, bt[:B2].contiguous(), sl[:B2].contiguous())
    _, acc1, m1, l1 = partial(big, ns)
    _, acc2, m2, l2 = partial(small, ns)
    assert torch.equal(acc1[:B2], acc2) and torch.equal(m1[:B2], m2) and torch.equal(l1[:B2], l2)


@pytest.mark.parametrize("ns", [4, 8, 33])
def test_fused_equals_two_launches(gpu, ns):
    Hq, Hkv = 16, 4
    B = -(-cus() // Hkv)
    case = make_case(lengths(B, seed=ns), Hq, Hkv, 16, pool_factor=1.25, seed=ns, poison=True)
    ws, n = fused_workspace(B, Hq, ns, case[0].device, fill=float("nan"))
    out = fused(case, ns, ws, n)
    ref2 = two_launch(case, ns)
    torch.cuda.synchronize()
    assert torch.equal(out, ref2), f"ns={ns}: fused != partial + merge bitwise"
    assert not counters(ws, B, Hq).any(), "arrival counters not left at zero"
    out2 = fused(case, ns, ws, n)
    torch.cuda.synchronize()
    assert torch.equal(out2, out)


@pytest.mark.parametrize("G,ns", [(4, 4), (4, 7), (4, 37), (4, 76), (4, 77), (4, 100), (3, 97),
                                  (2, 150), (1, 290), (1, 300)])
def test_v2_equals_partial_plus_merge(gpu, G, ns):
    """gqa_decode_v2_launch with one workgroup per pair merges the staged
    states inside the workgroup when every wave's splits fit its LDS stage
    (4-head groups: up to 19 splits a wave, so up to 76 splits; 3-head groups
    25, 2-head 37, 1-head 74), and runs the merge launch otherwise (the stage
    then also drains in mid-run): either way its output equals the partial
    launch followed by the merge launch bit for bit, and its workspace holds
    the partial launch's states. (3, 97) and (1, 290) merge in the workgroup
    with an odd number of staged floats per wave, whose LDS regions are padded
    to 16 bytes."""
    Hkv = 2
    B = -(-cus() // Hkv)
    case = make_case(lengths(B, seed=ns, top=6000), G * Hkv, Hkv, 16, pool_factor=1.25, seed=G,
                     poison=True)
    q, k, v, bt, sl = case
    Hq = q.shape[1]
    print(f"v2 vs partial+merge G={G} ns={ns} B={B}", flush=True)
    ws1, acc1, m1, l1 = partial(case, ns)
    ref = torch.empty_like(q)
    assert capi.v2_merge_launch(acc1.data_ptr(), m1.data_ptr(), l1.data_ptr(), ref.data_ptr(), B,
                                Hq, ns, stream_ptr()) == 0
    ws2, acc2, m2, l2 = alloc_ws(B, Hq, ns, q.device)
    ws2.fill_(float("nan"))
    out = torch.empty_like(q)
    assert capi.v2_launch(q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr(),
                          out.data_ptr(), B, Hq, Hkv, 16, bt.shape[1], SCALE, ns, acc2.data_ptr(),
                          m2.data_ptr(), l2.data_ptr(), stream_ptr()) == 0
    torch.cuda.synchronize()
    assert torch.equal(out, ref), f"G={G} ns={ns}: v2 != partial + merge bitwise"
    assert torch.equal(ws1, ws2), f"G={G} ns={ns}: v2's workspace != the partial launch's"
    check_states(case, acc1, m1, l1, ns, [0, 1, 2, 3, 9, B - 1])
    assert_close(out, oracle(case, SCALE), 2e-2, 2e-2, f"v2 G={G} ns={ns}")


@pytest.mark.parametrize("mode", ["merge_in_workgroup", "merge_launch", "fused"])
def test_graph_replay(gpu, mode):
    """The split-range launches captured in a HIP graph and replayed (new
    queries written between replays, the eager launch in between): every
    replay equals the eager launch bit for bit. merge_in_workgroup: one
    workgroup per pair, v2 is one kernel; merge_launch: two workgroups per
    pair, the partial kernel then the merge kernel; fused: the single-launch
    entry point on a one-workgroup-per-pair batch. Nothing here records a
    memset or allocates."""
    Hq, Hkv = 8, 2
    if mode == "merge_launch":
        B, ns = cus() // (Hkv * 2), 16  # 2 workgroups per pair, 16 >= 4 * 2 splits
        assert groups_per_pair(B, Hkv) == 2
    else:
        B, ns = -(-cus() // Hkv), 12
        assert groups_per_pair(B, Hkv) == 1
    case = make_case(lengths(B, seed=40), Hq, Hkv, 16, pool_factor=1.25, seed=41, poison=True)
    q, k, v, bt, sl = case
    ptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr())

    def make_launch(out):
        if mode == "fused":
            ws, n = fused_workspace(B, Hq, ns, q.device)
            return lambda: capi.v2_fused_launch(*ptrs, out.data_ptr(), B, Hq, Hkv, 16, bt.shape[1],
                                                SCALE, ns, ws.data_ptr(), n,
                                                torch.cuda.current_stream().cuda_stream)
        _, acc, m, l = alloc_ws(B, Hq, ns, q.device)
        return lambda: capi.v2_launch(*ptrs, out.data_ptr(), B, Hq, Hkv, 16, bt.shape[1], SCALE,
                                      ns, acc.data_ptr(), m.data_ptr(), l.data_ptr(),
                                      torch.cuda.current_stream().cuda_stream)

    out = torch.empty_like(q)
    launch = make_launch(out)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        assert launch() == 0  # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        assert launch() == 0
    eager_out = torch.empty_like(q)
    eager = make_launch(eager_out)
    gen = torch.Generator(device="cpu").manual_seed(42)
    for rep in range(4):
        q.copy_(torch.randn(q.shape, generator=gen).to(q.device, torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        assert eager() == 0
        torch.cuda.synchronize()
        assert torch.equal(out, eager_out), f"{mode}: replay {rep} differs from the eager launch"
    assert_close(out, oracle(case, SCALE), 2e-2, 2e-2, f"{mode}/graph")


def test_largest_split_count(gpu):
    """512 splits (GQA_DECODE_MAX_SPLITS) over one workgroup per pair: 128
    splits per wave, so each wave's LDS stage (19 states for 4-head groups)
    drains six times in mid-run, and the merge launch folds 512 states per
    row in batches of 64. Against partial + merge (bitwise) and the oracle;
    splits past the requests' ends hold the neutral state."""
    Hq, Hkv, ns = 16, 4, 512
    B = -(-cus() // Hkv)
    case = make_case(lengths(B, seed=512, top=20000), Hq, Hkv, 16, pool_factor=1.25, seed=5,
                     poison=True)
    q, k, v, bt, sl = case
    ws1, acc1, m1, l1 = partial(case, ns)
    check_states(case, acc1, m1, l1, ns, [0, 1, 5, 11])
    ref = torch.empty_like(q)
    assert capi.v2_merge_launch(acc1.data_ptr(), m1.data_ptr(), l1.data_ptr(), ref.data_ptr(), B,
                                Hq, ns, stream_ptr()) == 0
    out = gqa_decode_v2(*case, SCALE, num_splits=ns)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert_close(out, oracle(case, SCALE), 2e-2, 2e-2, "ns512")
