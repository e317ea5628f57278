"""GPU parity of the MLA absorbed-path decode kernel (include/mla_decode.h)
against the CPU oracle (oracle/mla_decode_oracle.c, pinned by
tests/test_mla_oracle.py).

The reference has no MLA kernel or tests of its own; its baseline's test grid
(FlashMLA at 15f13e5, whose parameters the reference logs in
docs/g0/flashmla_bench_raw.txt) sets the cases: s_q 1 and 2, h_q from 1 to 128
with one latent head, d = 576, dv = 512, block 64, uniform and varlen
lengths, causal and not, zero-length requests; inputs N(0,1) bf16 with NaN in
every cache slot a request must not read. Added: split counts 1..8 and the
automatic one, block sizes off the 32-token tile (the per-lane gather),
query-row counts that are not multiples of 32 or exceed one 128-row group,
bitwise repeatability, the FlashMLA-style Python surface, and a full-size
benchmark batch checked on a subset of requests. Tolerance: out within
atol = rtol = 2e-2 of the fp32 oracle (softmax weights are rounded to bf16
for the PV product, as in the GQA matrix-core scan), lse within 5e-3.
"""

import numpy as np
import pytest
import torch

import capi
from cases import MLA_CONFIGS, make_mla_case, mla_seq_lens
from mla import flash_mla_with_kvcache, get_mla_metadata
from oracle import c_oracle

pytestmark = pytest.mark.gpu

SCALE = 576 ** -0.5
ATOL = RTOL = 2e-2
LSE_ATOL = 5e-3


def host(t):
    return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16) \
        if t.dtype == torch.bfloat16 else t.cpu().numpy()


def oracle(case, causal, batches=None):
    q, kv, bt, sl = case
    qh, bth, slh = host(q), host(bt), host(sl)
    if batches is not None:
        qh, bth, slh = qh[batches], bth[batches], slh[batches]
    return c_oracle.mla_decode_ref(qh, host(kv), bth, slh, SCALE, causal=causal)


def run(case, causal, ns):
    q, kv, bt, sl = case
    B, s_q, h_q, _ = q.shape
    out = torch.empty(B, s_q, h_q, 512, dtype=torch.bfloat16, device=q.device)
    lse = torch.empty(B, h_q, s_q, dtype=torch.float32, device=q.device)
    wsb = capi.mla_workspace_bytes(B, s_q, h_q, ns)
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=q.device)
    rc = capi.mla_launch(q.data_ptr(), kv.data_ptr(), bt.data_ptr(), sl.data_ptr(), out.data_ptr(),
                         lse.data_ptr(), B, s_q, h_q, kv.shape[1], bt.shape[1], SCALE,
                         int(causal), ns, ws.data_ptr(), wsb, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    return out, lse


def check(got, want, label, rows=None):
    out, lse = got
    wo, wl = want
    o = out.float().cpu().numpy()
    l = lse.cpu().numpy()
    if rows is not None:
        o, l = o[rows], l[rows]
    bad = ~np.isclose(o, wo, atol=ATOL, rtol=RTOL)
    assert not bad.any(), f"{label}: out mismatch {bad.sum()} of {bad.size}, max-abs " \
                          f"{np.nanmax(np.abs(o - wo)):.3e}"
    assert (np.isneginf(l) == np.isneginf(wl)).all(), f"{label}: empty-row lse differs"
    fin = np.isfinite(wl)
    assert np.abs(l[fin] - wl[fin]).max(initial=0) <= LSE_ATOL, \
        f"{label}: lse max-abs {np.abs(l[fin] - wl[fin]).max():.3e}"


def mla_case(S_list, s_q, h_q, bs=64, seed=0):
    return make_mla_case(S_list, s_q, h_q, bs, pool_factor=2, seed=seed, device="cuda",
                         poison=True)


@pytest.mark.parametrize("s_q", [1, 2])
@pytest.mark.parametrize("h_q", [1, 16, 64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("varlen", [False, True])
def test_flashmla_grid(gpu, s_q, h_q, causal, varlen):
    S_list = mla_seq_lens(4, 700, seed=h_q, s_q=s_q) if varlen else [700] * 4
    print(f"mla s_q={s_q} h_q={h_q} causal={causal} varlen={varlen}", flush=True)
    case = mla_case(S_list, s_q, h_q, seed=h_q + s_q)
    want = oracle(case, causal)
    for ns in (1, 3, capi.mla_pick_num_splits(4, s_q, h_q, 64, case[2].shape[1], 0)):
        check(run(case, causal, ns), want, f"s_q{s_q}/h{h_q}/c{causal}/v{varlen}/ns{ns}")


@pytest.mark.parametrize("S_list", [[20], [1, 64, 65, 33], [0, 45, 0, 130]])
@pytest.mark.parametrize("ns", [1, 2, 8])
def test_short_and_empty(gpu, S_list, ns):
    # One token, exact and partial tiles, and zero-length requests (out 0,
    # lse -inf), with causal rows that see no key.
    case = mla_case(S_list, 2, 16, seed=len(S_list) + ns)
    for causal in (False, True):
        check(run(case, causal, ns), oracle(case, causal), f"{S_list}/ns{ns}/c{causal}")


@pytest.mark.parametrize("bs", [16, 32, 128, 7, 48])
def test_block_sizes(gpu, bs):
    # Multiples of 32 keep a tile inside one block (scalar block id); others
    # take the per-lane gather.
    case = mla_case([1, 200, 333, 64], 1, 64, bs=bs, seed=bs)
    for ns in (1, 4):
        check(run(case, False, ns), oracle(case, False), f"bs{bs}/ns{ns}")


@pytest.mark.parametrize("h_q", [3, 9, 33, 63, 65, 127, 200, 256])
def test_row_counts(gpu, h_q):
    # Row counts off the 32-row wave and past one 128-row group.
    case = mla_case([300, 1, 129], 1, h_q, seed=h_q)
    for ns in (1, 2):
        check(run(case, False, ns), oracle(case, False), f"h{h_q}/ns{ns}")


def test_bitwise_repeatable(gpu):
    case = mla_case(mla_seq_lens(8, 2000, seed=3), 1, 128, seed=3)
    for ns in (1, 4):
        first = run(case, False, ns)
        for _ in range(3):
            again = run(case, False, ns)
            assert torch.equal(again[0], first[0]) and torch.equal(again[1], first[1])


def test_python_surface(gpu):
    # FlashMLA-style calls: metadata, then the decode with the default scale.
    case = mla_case(mla_seq_lens(6, 1500, seed=4, s_q=2), 2, 32, seed=4)
    q, kv, bt, sl = case
    meta, splits = get_mla_metadata(sl, 2 * 32, 1)
    assert splits.shape == (7,) and int(meta[0, 0]) >= 1
    out, lse = flash_mla_with_kvcache(q, kv, bt, sl, 512, meta, splits, causal=True)
    torch.cuda.synchronize()
    check((out, lse), oracle(case, True), "flash_mla_with_kvcache")
    with pytest.raises(ValueError):
        flash_mla_with_kvcache(q.float(), kv, bt, sl, 512)
    with pytest.raises(ValueError):
        flash_mla_with_kvcache(q, kv, bt, sl, 256)


def test_benchmark_batch(gpu):
    # The mla_4k benchmark batch at full size (128 requests of ~4096 tokens,
    # 128 heads), checked against the oracle on 8 of its requests.
    cfg = MLA_CONFIGS["mla_4k"]
    S_list = mla_seq_lens(cfg["B"], cfg["S_mean"], seed=0)
    case = make_mla_case(S_list, cfg["s_q"], cfg["h_q"], cfg["bs"], pool_factor=1.1, seed=0,
                         device="cuda")
    ns = capi.mla_pick_num_splits(cfg["B"], 1, 128, 64, case[2].shape[1], 0)
    rows = [0, 17, 40, 63, 64, 99, 120, 127]
    check(run(case, False, ns), oracle(case, False, rows), "mla_4k", rows=rows)
