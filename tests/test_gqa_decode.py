"""GPU parity tests of the HIP kernels against the CPU oracle.

Mirrors the reference's tests/test_gqa_decode.py: its case grid (:89-98) on
each kernel, the num_splits sweep with the bitwise v2(ns=1) == v1 assertion
(:109-121), empty splits (:124-128) and large logits (:131-139), with its
inputs (0.5 * N(0,1), shuffled 2x pool, NaN in every slot that must not be
read, -1 padding) and its tolerance (atol = rtol = 2e-2, :22-23). Added:
run-to-run bitwise determinism, block sizes that are not multiples of 16
(the per-lane gather path), GQA group sizes 1..32, the split workspace
checked state by state against the oracle, the merge entry point on its own,
caller-owned workspace through the C ABI, and a non-default stream.
"""

import math

import numpy as np
import pytest
import torch

import capi
from binding import KERNELS, gqa_decode_v1, gqa_decode_v2
from cases import make_case
from gpu_util import assert_close, host_case, numpy_oracle, oracle
from oracle import reference as ref

pytestmark = pytest.mark.gpu

ATOL = 2e-2
RTOL = 2e-2
D = 128
SCALE = 1.0 / math.sqrt(D)

CASES = {
    "a_base": dict(S_list=[100, 257, 512, 33], Hq=32, Hkv=8, bs=16),
    "b_long": dict(S_list=[1000], Hq=32, Hkv=8, bs=16),
    "c_len1": dict(S_list=[1], Hq=32, Hkv=8, bs=16),
    "d_exact_blocks": dict(S_list=[16, 64], Hq=32, Hkv=8, bs=16),
    "e_partial_blocks": dict(S_list=[17, 65], Hq=32, Hkv=8, bs=16),
    "f_bs64": dict(S_list=[100, 257, 512, 33], Hq=32, Hkv=8, bs=64),
    "g_hq64": dict(S_list=[100, 257, 512, 33], Hq=64, Hkv=8, bs=16),
    "i_8k": dict(S_list=[8192, 8192], Hq=32, Hkv=8, bs=16),
}


def ref_case(cfg, seed=0, **kw):
    """The reference harness's inputs: 0.5*N(0,1), 2x pool, NaN poisoning."""
    S = cfg["S_list"]
    nb = sum((s + cfg["bs"] - 1) // cfg["bs"] for s in S)
    return make_case(S, cfg["Hq"], cfg["Hkv"], cfg["bs"], pool=2 * nb, seed=seed, qkv_std=0.5,
                     poison=True, **kw)


def run_and_check(fn, case, scale=SCALE, atol=ATOL, rtol=RTOL, label="", want=None):
    out = fn(*case, scale)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16 and out.shape == case[0].shape
    if want is None:
        want = numpy_oracle(case, scale)
    assert_close(out, want, atol, rtol, label)
    return out


@pytest.mark.parametrize("name", list(CASES))
@pytest.mark.parametrize("kernel", list(KERNELS))
def test_gqa_decode(gpu, kernel, name):
    print(f"case {name} kernel {kernel}", flush=True)
    run_and_check(KERNELS[kernel], ref_case(CASES[name]), label=f"{kernel}/{name}")


@pytest.mark.parametrize("num_splits", [1, 3, 8, 32])
def test_v2_num_splits(gpu, num_splits):
    case = ref_case(CASES["a_base"])
    run_and_check(lambda *a: gqa_decode_v2(*a, num_splits=num_splits), case)
    if num_splits == 1:
        # One split: the merge factor is exactly 1 and both paths share the
        # scan and the final division, so the outputs are bitwise equal.
        out_v2 = gqa_decode_v2(*case, SCALE, num_splits=1)
        out_v1 = gqa_decode_v1(*case, SCALE)
        assert torch.equal(out_v2, out_v1), "v2(num_splits=1) != v1 bitwise"


def test_v2_len1_splits8(gpu):
    # S=1 with 8 splits: 7 empty segments must contribute factor 0.
    run_and_check(lambda *a: gqa_decode_v2(*a, num_splits=8), ref_case(CASES["c_len1"]))


@pytest.mark.parametrize("kernel", list(KERNELS))
def test_gqa_decode_large_logits(gpu, kernel):
    q, k, v, bt, sl = ref_case(CASES["a_base"])
    q = (q.float() * 50.0).to(torch.bfloat16)
    out = run_and_check(KERNELS[kernel], (q, k, v, bt, sl))
    assert torch.isfinite(out.float()).all()


@pytest.mark.parametrize("kernel,ns", [("v1", None), ("v2", 1), ("v2", 7), ("v2", 64),
                                       ("v0", None)])
def test_bitwise_deterministic(gpu, kernel, ns):
    case = ref_case(CASES["a_base"])
    fn = KERNELS[kernel] if ns is None else (lambda *a: gqa_decode_v2(*a, num_splits=ns))
    first = fn(*case, SCALE)
    for _ in range(5):
        assert torch.equal(fn(*case, SCALE), first)


@pytest.mark.parametrize("bs", [1, 7, 8, 24, 32, 48, 128])
def test_block_sizes(gpu, bs):
    """Block sizes off the 16-token tile use the per-lane gather path."""
    cfg = dict(S_list=[1, 5, 33, 130, 611], Hq=32, Hkv=8, bs=bs)
    case = ref_case(cfg, seed=bs)
    want = numpy_oracle(case, SCALE)
    for kernel, fn in [("v1", gqa_decode_v1), ("v2", lambda *a: gqa_decode_v2(*a, num_splits=5)),
                       ("v0", KERNELS["v0"])]:
        run_and_check(fn, case, want=want, label=f"{kernel}/bs{bs}")


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (16, 8), (24, 8), (40, 8), (96, 8), (128, 8),
                                    (32, 1), (4, 2)])
def test_group_sizes(gpu, Hq, Hkv):
    cfg = dict(S_list=[77, 300, 16], Hq=Hq, Hkv=Hkv, bs=16)
    case = ref_case(cfg, seed=Hq + Hkv)
    want = numpy_oracle(case, SCALE)
    for kernel, fn in [("v1", gqa_decode_v1), ("v2", lambda *a: gqa_decode_v2(*a, num_splits=3)),
                       ("v0", KERNELS["v0"])]:
        run_and_check(fn, case, want=want, label=f"{kernel}/G{Hq // Hkv}")


def build_segments(S, ns, tile=32):
    """The partial kernel's documented segment rule: chunk = ceil(S/ns)
    rounded up to a multiple of 32 tokens."""
    chunk = -(-(-(-S // ns)) // tile) * tile
    return [(min(i * chunk, S), min(S, min(i * chunk, S) + chunk)) for i in range(ns)]


def alloc_ws(B, Hq, ns, device):
    states = B * Hq * ns
    ws = torch.empty(states * (D + 2), dtype=torch.float32, device=device)
    assert ws.numel() * 4 == capi.workspace_bytes(B, Hq, ns)
    return ws, ws[:states * D].view(B, Hq, ns, D), ws[states * D:states * (D + 1)].view(
        B, Hq, ns), ws[states * (D + 1):].view(B, Hq, ns)


def stream_ptr():
    return torch.cuda.current_stream().cuda_stream


# Relative error allowed per softmax weight in a state's l and acc: fp32
# scores and exponentials (~1e-6), the matrix-core scan's two-part bf16 weights
# (P_hi + P_lo, within 2^-18 of the fp32 weight) and fp32 summation over a
# segment. A single bf16 part per weight (2^-9) would exceed it.
W_REL = 1e-4


@pytest.mark.parametrize("ns", [1, 4, 9])
def test_partial_states_match_oracle(gpu, ns):
    """Each (b, q-head, split) workspace state against the oracle's state of
    the same token range: m in natural-log units, l, and unnormalised acc."""
    cfg = dict(S_list=[1, 40, 333, 16], Hq=16, Hkv=4, bs=16)
    case = ref_case(cfg, seed=11)
    q, k, v, bt, sl = case
    B, Hq = q.shape[:2]
    ws, acc, m, l = alloc_ws(B, Hq, ns, q.device)
    ws.fill_(float("nan"))
    rc = capi.v2_partial_launch(q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(),
                                sl.data_ptr(), B, Hq, 4, 16, bt.shape[1], SCALE, ns,
                                acc.data_ptr(), m.data_ptr(), l.data_ptr(), stream_ptr())
    assert rc == 0
    torch.cuda.synchronize()
    qh, kh, vh, bth, slh = host_case(case)
    acc_h, m_h, l_h = acc.cpu().numpy(), m.cpu().numpy(), l.cpu().numpy()
    for b in range(B):
        K, V = ref.gather_kv(kh, vh, bth, int(slh[b]), b)
        for h in range(Hq):
            for i, (a, e) in enumerate(build_segments(int(slh[b]), ns)):
                mw, lw, aw = ref.partial_state(ref.bf16_to_f32(qh[b, h]), K[a:e, h // 4],
                                               V[a:e, h // 4], SCALE)
                if a == e:
                    assert m_h[b, h, i] == -np.inf and l_h[b, h, i] == 0
                    assert not acc_h[b, h, i].any()
                    continue
                assert m_h[b, h, i] == pytest.approx(mw, abs=1e-5)
                assert l_h[b, h, i] == pytest.approx(lw, rel=W_REL)
                # |acc error| <= W_REL * sum_t p_t |v_t| <= W_REL * l * max|v|
                vmax = float(np.abs(V[a:e, h // 4]).max())
                np.testing.assert_allclose(acc_h[b, h, i], aw, rtol=0, atol=W_REL * lw * vmax)


def test_merge_entry_point(gpu):
    """The merge kernel alone, fed oracle states (including empty splits)."""
    rng = np.random.default_rng(0)
    B, Hq, ns = 3, 8, 6
    m = rng.standard_normal((B, Hq, ns)) * 3
    m[0, :, 2:] = -np.inf  # empty splits
    l = np.where(m == -np.inf, 0.0, rng.uniform(0.5, 20, (B, Hq, ns)))
    acc = rng.standard_normal((B, Hq, ns, D)) * l[..., None]
    acc[m == -np.inf] = 0
    dev = torch.device("cuda")
    t = [torch.tensor(x, dtype=torch.float32, device=dev).contiguous() for x in (acc, m, l)]
    out = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=dev)
    assert capi.v2_merge_launch(t[0].data_ptr(), t[1].data_ptr(), t[2].data_ptr(),
                                out.data_ptr(), B, Hq, ns, stream_ptr()) == 0
    torch.cuda.synchronize()
    want = np.stack([np.stack([ref.merge_states(m[b, h], l[b, h], acc[b, h])[0]
                               for h in range(Hq)]) for b in range(B)])
    assert_close(out, want, 1e-2, 1e-2, "merge")


@pytest.mark.parametrize("ranks", [2, 3])
def test_context_parallel_shards(gpu, ranks):
    """Sharding by tokens (context parallelism) on one GPU: each "rank" holds a
    contiguous range of every request's blocks -- its own block table and
    lengths, possibly empty -- and computes one state per (request, q-head)
    with the exported partial launch; the states, placed in rank order as an
    all-gather delivers them, go through the exported merge launch. The result
    matches the oracle on the whole sequences."""
    S_list, Hq, Hkv, bs = [3000, 517, 1, 2048, 40], 32, 8, 16
    case = ref_case(dict(S_list=S_list, Hq=Hq, Hkv=Hkv, bs=bs), seed=31)
    q, k, v, bt, sl = case
    B = q.shape[0]
    bt_h = bt.cpu()
    accs, ms, ls = [], [], []
    for r in range(ranks):
        lens, rows = [], []
        for b, S in enumerate(S_list):
            nb = (S + bs - 1) // bs
            lo, hi = r * nb // ranks, (r + 1) * nb // ranks
            lens.append(max(0, min(S, hi * bs) - lo * bs))
            rows.append(bt_h[b, lo:hi])
        mb = max(1, max(len(x) for x in rows))
        bt_r = torch.full((B, mb), -1, dtype=torch.int32)
        for b, x in enumerate(rows):
            bt_r[b, :len(x)] = x
        bt_r = bt_r.to(q.device)
        sl_r = torch.tensor(lens, dtype=torch.int32, device=q.device)
        _, acc, m, l = alloc_ws(B, Hq, 1, q.device)
        assert capi.v2_partial_launch(q.data_ptr(), k.data_ptr(), v.data_ptr(), bt_r.data_ptr(),
                                      sl_r.data_ptr(), B, Hq, Hkv, bs, mb, SCALE, 1,
                                      acc.data_ptr(), m.data_ptr(), l.data_ptr(),
                                      stream_ptr()) == 0
        accs.append(acc)
        ms.append(m)
        ls.append(l)
    acc_all = torch.cat(accs, dim=2).contiguous()  # [B, Hq, ranks, D]
    m_all = torch.cat(ms, dim=2).contiguous()
    l_all = torch.cat(ls, dim=2).contiguous()
    out = torch.empty_like(q)
    assert capi.v2_merge_launch(acc_all.data_ptr(), m_all.data_ptr(), l_all.data_ptr(),
                                out.data_ptr(), B, Hq, ranks, stream_ptr()) == 0
    torch.cuda.synchronize()
    assert_close(out, numpy_oracle(case, SCALE), ATOL, RTOL, f"cp{ranks}")


def test_capi_v2_matches_op(gpu):
    case = ref_case(CASES["a_base"])
    q, k, v, bt, sl = case
    B, Hq = q.shape[:2]
    ns = 5
    ws, acc, m, l = alloc_ws(B, Hq, ns, q.device)
    out = torch.empty_like(q)
    rc = capi.v2_launch(q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr(),
                        out.data_ptr(), B, Hq, 8, 16, bt.shape[1], SCALE, ns, acc.data_ptr(),
                        m.data_ptr(), l.data_ptr(), stream_ptr())
    assert rc == 0
    assert torch.equal(out, gqa_decode_v2(*case, SCALE, num_splits=ns))
    out1 = torch.empty_like(q)
    assert capi.v1_launch(q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr(),
                          out1.data_ptr(), B, Hq, 8, 16, bt.shape[1], SCALE, stream_ptr()) == 0
    assert torch.equal(out1, gqa_decode_v1(*case, SCALE))


def test_v2_one_split_writes_workspace(gpu):
    """v2 with one split runs the single-pass kernel, which still fills the
    caller's workspace with the one-split state."""
    case = ref_case(CASES["a_base"])
    q, k, v, bt, sl = case
    B, Hq = q.shape[:2]
    ws1, acc1, m1, l1 = alloc_ws(B, Hq, 1, q.device)
    ws2, acc2, m2, l2 = alloc_ws(B, Hq, 1, q.device)
    ws1.fill_(float("nan"))
    out = torch.empty_like(q)
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr())
    assert capi.v2_launch(*args, out.data_ptr(), B, Hq, 8, 16, bt.shape[1], SCALE, 1,
                          acc1.data_ptr(), m1.data_ptr(), l1.data_ptr(), stream_ptr()) == 0
    assert capi.v2_partial_launch(*args, B, Hq, 8, 16, bt.shape[1], SCALE, 1, acc2.data_ptr(),
                                  m2.data_ptr(), l2.data_ptr(), stream_ptr()) == 0
    torch.cuda.synchronize()
    assert torch.equal(ws1, ws2)
    assert torch.equal(out, gqa_decode_v1(*case, SCALE))


def test_current_stream_is_used(gpu):
    case = ref_case(CASES["a_base"])
    want = gqa_decode_v2(*case, SCALE, num_splits=4)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        out = gqa_decode_v2(*case, SCALE, num_splits=4)
        out1 = gqa_decode_v1(*case, SCALE)
    s.synchronize()
    assert torch.equal(out, want)
    assert torch.equal(out1, gqa_decode_v2(*case, SCALE, num_splits=1))


@pytest.mark.parametrize("scale", [1.0, 0.01, SCALE * 3])
def test_scales(gpu, scale):
    case = ref_case(CASES["a_base"])
    run_and_check(lambda *a: gqa_decode_v2(*a, num_splits=0), case, scale=scale)


def test_heuristic_num_splits(gpu):
    case = ref_case(CASES["i_8k"])
    run_and_check(lambda *a: gqa_decode_v2(*a, num_splits=0), case)


@pytest.mark.parametrize("max_blocks", [32, 33])
def test_op_automatic_choice_short_sequences(gpu, max_blocks):
    # The op's automatic choice takes one split for block tables of at most
    # 512 tokens (output bitwise v1's), where the C ABI's heuristic gives 4
    # (config 1's shape); one more block and the heuristic's count runs.
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    S = [500, 512] if max_blocks == 32 else [500, 528]
    case = make_case(S, 32, 8, 16, pool_factor=1.25, seed=max_blocks, max_blocks=max_blocks)
    ns = capi.pick_num_splits(2, 32, 8, 16, max_blocks, cus)
    assert ns > 1
    out = gqa_decode_v2(*case, SCALE, num_splits=0)
    want = gqa_decode_v1(*case, SCALE) if max_blocks == 32 else \
        gqa_decode_v2(*case, SCALE, num_splits=ns)
    assert torch.equal(out, want)
    assert_close(out, oracle(case, SCALE), 2e-2, 2e-2, f"auto, max_blocks={max_blocks}")


def test_op_input_errors_on_device(gpu):
    q, k, v, bt, sl = ref_case(CASES["a_base"])
    with pytest.raises(RuntimeError, match="Hq must be divisible by Hkv"):
        gqa_decode_v1(q[:, :30].contiguous(), k, v, bt, sl, SCALE)
    with pytest.raises(RuntimeError, match="num_splits must be in"):
        gqa_decode_v2(q, k, v, bt, sl, SCALE, num_splits=513)
    with pytest.raises(RuntimeError, match="block_table must be int32"):
        gqa_decode_v1(q, k, v, bt.long(), sl, SCALE)
    with pytest.raises(RuntimeError, match="k_cache and v_cache must have the same shape"):
        gqa_decode_v1(q, k, v[:-1], bt, sl, SCALE)
