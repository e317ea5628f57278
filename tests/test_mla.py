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
bitwise repeatability, the FlashMLA-style Python surface, a full-size
benchmark batch checked on a subset of requests, and exact properties of
whole benchmark batches with no oracle in the loop (twice the cache with half
the scale: twice out and the same lse, bit for bit; every output between its
value rows' extremes). Tolerance: out within
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


def oracle(case, causal, batches=None, scale=SCALE):
    q, kv, bt, sl = case
    qh, bth, slh = host(q), host(bt), host(sl)
    if batches is not None:
        qh, bth, slh = qh[batches], bth[batches], slh[batches]
    return c_oracle.mla_decode_ref(qh, host(kv), bth, slh, scale, causal=causal)


def run(case, causal, ns, scale=SCALE):
    q, kv, bt, sl = case
    B, s_q, h_q, _ = q.shape
    out = torch.empty(B, s_q, h_q, 512, dtype=torch.bfloat16, device=q.device)
    lse = torch.empty(B, h_q, s_q, dtype=torch.float32, device=q.device)
    wsb = capi.mla_workspace_bytes(B, s_q, h_q, ns)
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=q.device)
    rc = capi.mla_launch(q.data_ptr(), kv.data_ptr(), bt.data_ptr(), sl.data_ptr(), out.data_ptr(),
                         lse.data_ptr(), B, s_q, h_q, kv.shape[1], bt.shape[1], scale,
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


@pytest.mark.parametrize("bs", [16, 32, 128, 7, 48, 1, 3])
def test_block_sizes(gpu, bs):
    # Multiples of 32 keep a tile inside one block (scalar block id); others
    # take the per-lane gather (block 1: a tile spans 32 blocks).
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
    want = oracle(case, True)
    meta, splits = get_mla_metadata(sl, 2 * 32, 1)
    assert meta.device.type == "cpu" and int(meta[0, 0]) == 0 and int(meta[0, 1]) > 0
    assert splits.shape == (7,) and int(splits[-1]) >= int((sl > 0).sum())
    out, lse = flash_mla_with_kvcache(q, kv, bt, sl, 512, meta, splits, causal=True)
    torch.cuda.synchronize()
    check((out, lse), want, "flash_mla_with_kvcache balanced")
    for n in (0, 3):
        meta, splits = get_mla_metadata(sl, 2 * 32, 1, num_splits=n)
        assert int(meta[0, 0]) >= 1
        out, lse = flash_mla_with_kvcache(q, kv, bt, sl, 512, meta, splits, causal=True)
        torch.cuda.synchronize()
        check((out, lse), want, f"flash_mla_with_kvcache splits={n}")
    out, lse = flash_mla_with_kvcache(q, kv, bt, sl, 512, causal=True)
    torch.cuda.synchronize()
    check((out, lse), want, "flash_mla_with_kvcache default")
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


@pytest.mark.parametrize("ns", [1, 2, 5])
def test_split_and_combine_launches(gpu, ns):
    # The two halves of mla_decode_launch, launched apart, give its bits.
    case = mla_case(mla_seq_lens(5, 900, seed=5, s_q=2), 2, 64, seed=5)
    q, kv, bt, sl = case
    B, s_q, h_q, _ = q.shape
    want = run(case, True, ns)
    out = torch.empty_like(want[0])
    lse = torch.empty_like(want[1])
    wsb = capi.mla_workspace_bytes(B, s_q, h_q, ns)
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=q.device)
    sp = torch.cuda.current_stream().cuda_stream
    assert capi.mla_splitkv_launch(q.data_ptr(), kv.data_ptr(), bt.data_ptr(), sl.data_ptr(),
                                   out.data_ptr(), lse.data_ptr(), B, s_q, h_q, kv.shape[1],
                                   bt.shape[1], SCALE, 1, ns, ws.data_ptr(), wsb, sp) == 0
    if ns > 1:
        assert capi.mla_combine_launch(ws.data_ptr(), wsb, out.data_ptr(), lse.data_ptr(), B, s_q,
                                       h_q, ns, sp) == 0
    torch.cuda.synchronize()
    assert torch.equal(out, want[0]) and torch.equal(lse, want[1])


@pytest.mark.parametrize("ranks", [2, 3])
def test_context_parallel_shards(gpu, ranks):
    # Sharding long requests by tokens across GPUs, on one GPU: each "rank"
    # holds a contiguous range of every request's blocks (its own block table
    # and lengths, some empty) and runs the split launch with 2 splits; the
    # workspace states, placed in rank order per (request, query row) as an
    # all-gather delivers them, go through the combine launch with 2 x ranks
    # splits. out and lse match the oracle on the whole sequences.
    S_list, s_q, h_q, bs = [2900, 450, 1, 1300, 64], 2, 32, 64
    case = mla_case(S_list, s_q, h_q, bs=bs, seed=41)
    q, kv, bt, sl = case
    B, R = len(S_list), s_q * h_q
    bt_h = bt.cpu()
    sp = torch.cuda.current_stream().cuda_stream
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
        wsb = capi.mla_workspace_bytes(B, s_q, h_q, 2)
        ws = torch.empty(wsb // 4, dtype=torch.float32, device=q.device)
        scratch_out = torch.empty(B, s_q, h_q, 512, dtype=torch.bfloat16, device=q.device)
        scratch_lse = torch.empty(B, h_q, s_q, dtype=torch.float32, device=q.device)
        assert capi.mla_splitkv_launch(q.data_ptr(), kv.data_ptr(), bt_r.data_ptr(),
                                       sl_r.data_ptr(), scratch_out.data_ptr(),
                                       scratch_lse.data_ptr(), B, s_q, h_q, bs, mb, SCALE, 0, 2,
                                       ws.data_ptr(), wsb, sp) == 0
        states = B * R * 2
        accs.append(ws[:states * 512].view(B * R, 2, 512))
        ms.append(ws[states * 512:states * 513].view(B * R, 2))
        ls.append(ws[states * 513:states * 514].view(B * R, 2))
    ns = 2 * ranks
    gathered = torch.cat([torch.cat(accs, dim=1).flatten(), torch.cat(ms, dim=1).flatten(),
                          torch.cat(ls, dim=1).flatten()])
    wsb = capi.mla_workspace_bytes(B, s_q, h_q, ns)
    assert gathered.numel() * 4 == wsb
    out = torch.empty(B, s_q, h_q, 512, dtype=torch.bfloat16, device=q.device)
    lse = torch.empty(B, h_q, s_q, dtype=torch.float32, device=q.device)
    assert capi.mla_combine_launch(gathered.data_ptr(), wsb, out.data_ptr(), lse.data_ptr(), B,
                                   s_q, h_q, ns, sp) == 0
    torch.cuda.synchronize()
    check((out, lse), oracle(case, False), f"cp{ranks}")


@pytest.mark.parametrize("ns", [1, 3])
def test_late_dominant_key(gpu, ns):
    # A key far above everything before it (score ~ 2|q|^2, ~70 in log2
    # units above the first tiles' maxima, past the 32-unit slack of the
    # first-tile reference but not past fp32's range): the workgroup runs its
    # split a second time against the true maxima. Other rows get a dominant
    # key in their first tile (no second pass needed), and request 1 none at
    # all. test_overflowing_late_key plants keys that would overflow without
    # the second pass.
    case = mla_case([700, 300, 95], 1, 64, seed=11)
    q, kv, bt, sl = case
    bs = kv.shape[1]
    for row, tok in ((5, 400), (40, 690), (63, 33)):
        blk, slot = int(bt[0, tok // bs]), tok % bs
        kv[blk, slot, 0] = (q[0, 0, row].float() * 2).to(torch.bfloat16)
    blk = int(bt[2, 2 // bs])
    kv[blk, 2 % bs, 0] = (q[2, 0, 7].float() * 2).to(torch.bfloat16)
    for causal in (False, True):
        check(run(case, causal, ns), oracle(case, causal), f"dominant/ns{ns}/c{causal}")


# Keys 5 q (score 5 |q|^2 / 24, ~170 log2 units) planted at (row, token) of
# request 0, in rows other than row 0 of their 16-row MFMA block and at tokens
# outside lane 0's score slots (lane (j, g) holds row j's tokens 16 tg + 4 g +
# e of a tile): a restart vote read from lane 0 alone would miss all of them.
OVERFLOW_PLANTS = ((5, 405), (40, 694), (63, 45), (97, 301))


def overflow_case():
    case = mla_case([700, 300, 95], 1, 128, seed=13)
    q, kv, bt, sl = case
    bs = kv.shape[1]
    for row, tok in OVERFLOW_PLANTS:
        assert row % 16 != 0 and (tok % 16) // 4 != 0
        kv[int(bt[0, tok // bs]), tok % bs, 0] = (q[0, 0, row].float() * 5).to(torch.bfloat16)
    # Each planted score beats every other key of its row by more than 128
    # log2 units: against any reference not set by the planted key itself,
    # exp2 overflows fp32, so a finite, correct result needs the second pass.
    qh = q[0, 0].float().cpu().double().numpy()
    keys = torch.stack([kv[int(bt[0, t // bs]), t % bs, 0] for t in range(700)]).float()
    sc = (qh @ keys.cpu().double().numpy().T) * SCALE / np.log(2.0)
    for row, tok in OVERFLOW_PLANTS:
        assert sc[row, tok] - np.delete(sc[row], tok).max() > 128.0
    return case


def split_first_tile(tok, S, ns):
    """First tile (in tokens) of the fixed split holding token tok."""
    chunk = (-(-S // ns) + 31) // 32 * 32
    return tok // chunk * chunk


def share_first_tile(tok, tiles_before, T, n):
    """First tile (in tokens, request-relative) of the balanced piece holding
    token tok of a request whose tiles start at tiles_before."""
    n = min(n, T)
    t = tiles_before + tok // 32
    w = max(w for w in range(n) if w * T // n <= t)
    return (max(w * T // n, tiles_before) - tiles_before) * 32


@pytest.mark.parametrize("ns", [1, 3, 5])
def test_overflowing_late_key(gpu, ns):
    case = overflow_case()
    for _, tok in OVERFLOW_PLANTS:
        assert tok // 32 * 32 != split_first_tile(tok, 700, ns), "plant sets its reference"
    for causal in (False, True):
        got = run(case, causal, ns)
        assert torch.isfinite(got[0].float()).all()
        check(got, oracle(case, causal), f"overflow/ns{ns}/c{causal}")


# --------------------------------------------------------- token-balanced launch


def run_balanced(case, causal, nwg, scale=SCALE):
    q, kv, bt, sl = case
    B, s_q, h_q, _ = q.shape
    out = torch.empty(B, s_q, h_q, 512, dtype=torch.bfloat16, device=q.device)
    lse = torch.empty(B, h_q, s_q, dtype=torch.float32, device=q.device)
    wsb = capi.mla_balanced_workspace_bytes(B, s_q, h_q, nwg)
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=q.device)
    rc = capi.mla_balanced_launch(q.data_ptr(), kv.data_ptr(), bt.data_ptr(), sl.data_ptr(),
                                  out.data_ptr(), lse.data_ptr(), B, s_q, h_q, kv.shape[1],
                                  bt.shape[1], scale, int(causal), nwg, ws.data_ptr(), wsb,
                                  torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    return out, lse


@pytest.mark.parametrize("s_q", [1, 2])
@pytest.mark.parametrize("h_q", [16, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_balanced_flashmla_grid(gpu, s_q, h_q, causal):
    S_list = mla_seq_lens(6, 900, seed=h_q + 1, s_q=s_q)
    print(f"balanced s_q={s_q} h_q={h_q} causal={causal} S={S_list}", flush=True)
    case = mla_case(S_list, s_q, h_q, seed=h_q + s_q + 1)
    want = oracle(case, causal)
    for nwg in (1, 5, 64, 256):
        check(run_balanced(case, causal, nwg), want, f"bal s_q{s_q}/h{h_q}/c{causal}/n{nwg}")


@pytest.mark.parametrize("s_q", [3, 4, 8])
@pytest.mark.parametrize("h_q", [16, 128])
def test_more_query_tokens(gpu, s_q, h_q):
    # Beyond FlashMLA's benchmark grid: 3, 4 and 8 query tokens per request
    # (speculative decoding), causal and not, through both launches. With
    # h_q = 128 the rows span 3 to 8 row groups of 128; with causal masking
    # each query token's key limit differs by one, and the short requests
    # (down to s_q tokens) leave the first query tokens a single key.
    S_list = mla_seq_lens(5, 600, seed=s_q * h_q, s_q=s_q) + [s_q, s_q + 31]
    print(f"mla s_q={s_q} h_q={h_q} S={S_list}", flush=True)
    case = mla_case(S_list, s_q, h_q, seed=s_q + h_q)
    for causal in (False, True):
        want = oracle(case, causal)
        for ns in (1, 3):
            check(run(case, causal, ns), want, f"s_q{s_q}/h{h_q}/c{causal}/ns{ns}")
        for nwg in (7, 256):
            check(run_balanced(case, causal, nwg), want, f"bal s_q{s_q}/h{h_q}/c{causal}/n{nwg}")


@pytest.mark.parametrize("seed", range(12))
def test_random_shapes(gpu, seed):
    # Seeded random combinations the fixed grids above do not pair up: batch
    # 1-9, 1-4 query tokens, any head count 1-140, block sizes from 1 to 128
    # (multiples of 32 and not), lengths from 0 to 2500 (some shorter than
    # s_q, so that causal rows can have no key), causal or not; each through
    # fixed splits (1-6) and the balanced launch (1-300 shares).
    rng = np.random.RandomState(1000 + seed)
    B = int(rng.randint(1, 10))
    s_q = int(rng.randint(1, 5))
    h_q = int(rng.randint(1, 141))
    bs = int(rng.choice([1, 7, 16, 32, 48, 64, 96, 128]))
    S_list = [int(x) for x in rng.randint(0, 2501, size=B)]
    S_list[int(rng.randint(0, B))] = int(rng.randint(0, s_q + 1))
    causal = bool(rng.randint(0, 2))
    ns = int(rng.randint(1, 7))
    nwg = int(rng.randint(1, 301))
    print(f"mla random seed={seed}: B={B} s_q={s_q} h_q={h_q} bs={bs} causal={causal} "
          f"ns={ns} nwg={nwg} S={S_list}", flush=True)
    case = mla_case(S_list, s_q, h_q, bs=bs, seed=seed)
    want = oracle(case, causal)
    check(run(case, causal, ns), want, f"random{seed}/ns{ns}")
    check(run_balanced(case, causal, nwg), want, f"random{seed}/bal{nwg}")


def test_long_request(gpu):
    # One request of 65536 tokens with a short one beside it: the balanced
    # launch cuts it into ~256 pieces of ~8 tiles and the merge folds a few
    # hundred states per row; fixed splits take it at 64 and 128 (the most
    # accepted) splits.
    S_list = [65536, 300]
    print(f"mla long request S={S_list}", flush=True)
    case = mla_case(S_list, 1, 128, seed=61)
    for causal in (False, True):
        want = oracle(case, causal)
        check(run_balanced(case, causal, 256), want, f"long/c{causal}/bal256")
        for ns in (64, 128):
            check(run(case, causal, ns), want, f"long/c{causal}/ns{ns}")


@pytest.mark.parametrize("scale", [0.01, 0.2, 1.0])
def test_softmax_scales(gpu, scale):
    # softmax_scale other than 1/sqrt(576): small (nearly uniform weights over
    # every key) and large (scores spread over hundreds of log2 units, nearly
    # one-hot rows; rows whose later tiles beat their first tile's maximum by
    # more than the reference slack take the second pass).
    case = mla_case(mla_seq_lens(4, 800, seed=51, s_q=2), 2, 32, seed=51)
    for causal in (False, True):
        want = oracle(case, causal, scale=scale)
        check(run(case, causal, 3, scale=scale), want, f"scale{scale}/c{causal}/ns3")
        check(run_balanced(case, causal, 37, scale=scale), want,
              f"scale{scale}/c{causal}/bal37")


@pytest.mark.parametrize("S_list", [[0], [0, 0, 5], [1, 0, 64, 65, 0, 33], [3000], [31, 32, 33],
                                    [0, 2000, 0, 1, 700]])
def test_balanced_ragged_and_empty(gpu, S_list):
    # Empty requests, one-token requests, one long request over every share,
    # and share counts below, at and above the tile count.
    case = mla_case(S_list, 2, 16, seed=len(S_list))
    tiles = sum(-(-s // 32) for s in S_list)
    for causal in (False, True):
        want = oracle(case, causal)
        for nwg in sorted({1, 2, max(1, tiles), tiles + 3, 97}):
            check(run_balanced(case, causal, nwg), want, f"{S_list}/c{causal}/n{nwg}")


@pytest.mark.parametrize("bs", [16, 48, 128, 1])
def test_balanced_block_sizes(gpu, bs):
    case = mla_case([1, 200, 333, 64, 900], 1, 64, bs=bs, seed=bs + 1)
    want = oracle(case, False)
    for nwg in (3, 17):
        check(run_balanced(case, False, nwg), want, f"bal bs{bs}/n{nwg}")


@pytest.mark.parametrize("h_q", [33, 200, 256])
def test_balanced_row_groups(gpu, h_q):
    # Rows past one 128-row group: one set of shares per row group.
    case = mla_case([300, 1, 129, 500], 1, h_q, seed=h_q + 2)
    want = oracle(case, True)
    for nwg in (4, 24):
        check(run_balanced(case, True, nwg), want, f"bal h{h_q}/n{nwg}")


def test_balanced_repeatable_and_close_to_split(gpu):
    case = mla_case(mla_seq_lens(9, 1500, seed=8), 1, 128, seed=8)
    first = run_balanced(case, False, 40)
    for _ in range(3):
        again = run_balanced(case, False, 40)
        assert torch.equal(again[0], first[0]) and torch.equal(again[1], first[1])
    split = run(case, False, 4)
    assert torch.allclose(first[0].float(), split[0].float(), atol=2e-2, rtol=2e-2)
    fin = torch.isfinite(split[1])
    assert torch.allclose(first[1][fin], split[1][fin], atol=5e-3)


def test_balanced_late_dominant_key(gpu):
    case = mla_case([700, 300, 95], 1, 64, seed=11)
    q, kv, bt, sl = case
    bs = kv.shape[1]
    for row, tok in ((5, 400), (40, 690), (63, 33)):
        blk, slot = int(bt[0, tok // bs]), tok % bs
        kv[blk, slot, 0] = (q[0, 0, row].float() * 2).to(torch.bfloat16)
    want = oracle(case, False)
    for nwg in (1, 4, 9):
        check(run_balanced(case, False, nwg), want, f"bal dominant/n{nwg}")


def test_balanced_benchmark_batch(gpu):
    cfg = MLA_CONFIGS["mla_4k"]
    S_list = mla_seq_lens(cfg["B"], cfg["S_mean"], seed=0)
    case = make_mla_case(S_list, cfg["s_q"], cfg["h_q"], cfg["bs"], pool_factor=1.1, seed=0,
                         device="cuda")
    rows = [0, 17, 40, 63, 64, 99, 120, 127]
    check(run_balanced(case, False, 256), oracle(case, False, rows), "bal mla_4k", rows=rows)


def test_balanced_graph_replay(gpu):
    # The balanced launch (plan, split, merge: no host sync, no memset) inside a
    # HIP graph: every replay, with eager work between, equals the eager run.
    case = mla_case(mla_seq_lens(5, 800, seed=12, s_q=2), 2, 32, seed=12)
    q, kv, bt, sl = case
    B, s_q, h_q, _ = q.shape
    want = run_balanced(case, True, 24)
    out = torch.empty_like(want[0])
    lse = torch.empty_like(want[1])
    wsb = capi.mla_balanced_workspace_bytes(B, s_q, h_q, 24)
    ws = torch.empty(wsb, dtype=torch.uint8, device=q.device)
    s = torch.cuda.Stream()
    args = lambda st: (q.data_ptr(), kv.data_ptr(), bt.data_ptr(), sl.data_ptr(),  # noqa: E731
                       out.data_ptr(), lse.data_ptr(), B, s_q, h_q, kv.shape[1], bt.shape[1],
                       SCALE, 1, 24, ws.data_ptr(), wsb, st.cuda_stream)
    with torch.cuda.stream(s):
        assert capi.mla_balanced_launch(*args(s)) == 0  # warm-up on the capture stream
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        assert capi.mla_balanced_launch(*args(s)) == 0
    for rep in range(4):
        out.zero_()
        lse.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want[0]) and torch.equal(lse, want[1]), f"replay {rep}"
        run_balanced(case, False, 7)  # eager work between replays


def test_balanced_many_requests(gpu):
    # 3000 short requests (the split kernel's planning scan then takes several
    # requests per thread), checked on a subset.
    S_list = [(7 * i) % 97 for i in range(3000)]
    case = make_mla_case(S_list, 1, 16, 16, pool_factor=1.0, seed=13, device="cuda")
    got = run_balanced(case, False, 256)
    rows = [0, 1, 2, 500, 1499, 2998, 2999]
    check(got, oracle(case, False, rows), "bal many", rows=rows)


def test_balanced_overflowing_late_key(gpu):
    case = overflow_case()
    T = sum(-(-x // 32) for x in (700, 300, 95))
    want = oracle(case, False)
    for nwg in (1, 4, 9):
        for _, tok in OVERFLOW_PLANTS:
            assert tok // 32 * 32 != share_first_tile(tok, 0, T, nwg), "plant sets its reference"
        got = run_balanced(case, False, nwg)
        assert torch.isfinite(got[0].float()).all()
        check(got, want, f"bal overflow/n{nwg}")


def benchmark_case(name="mla_4k"):
    cfg = MLA_CONFIGS[name]
    S_list = mla_seq_lens(cfg["B"], cfg["S_mean"], seed=0, s_q=cfg["s_q"])
    return make_mla_case(S_list, cfg["s_q"], cfg["h_q"], cfg["bs"], pool_factor=1.1, seed=0,
                         device="cuda")


def launchers(case):
    ns = capi.mla_pick_num_splits(case[0].shape[0], case[0].shape[1], case[0].shape[2],
                                  case[1].shape[1], case[2].shape[1], 0)
    return {"split": lambda c, causal, s: run(c, causal, ns, s),
            "balanced": lambda c, causal, s: run_balanced(c, causal, 256, s)}


@pytest.mark.parametrize("name,causal", [("mla_4k", False), ("mla_4k_sq2", True)])
def test_cache_scale_property(gpu, name, causal):
    # A latent row is the key (576 dims) and the value (its first 512): twice
    # the cache with half the scale gives the same scores bit for bit (binary
    # floating point scales by 2 without rounding), so twice out and the same
    # lse, bit for bit, at the benchmark batch's full size, no oracle needed.
    case = benchmark_case(name)
    q, kv, bt, sl = case
    doubled = (q, kv * 2, bt, sl)
    for label, f in launchers(case).items():
        print(f"{name} cache scale {label}", flush=True)
        out, lse = f(case, causal, SCALE)
        out2, lse2 = f(doubled, causal, SCALE / 2)
        assert torch.equal(out2, out * 2), f"{name}/{label}: out(2C, scale/2) != 2 out(C, scale)"
        assert torch.equal(lse2, lse), f"{name}/{label}: lse changed"


def test_convex_combination(gpu):
    # out[b, i, h] is a convex combination of the request's value rows (the
    # first 512 dims of its latent rows): every element lies between their
    # smallest and largest value in that dimension (up to out's bf16 rounding).
    case = benchmark_case("mla_4k")
    q, kv, bt, sl = case
    bs = kv.shape[1]
    lo, hi = [], []
    for b, S in enumerate(sl.tolist()):
        nblk = -(-S // bs)
        rows = kv[bt[b, :nblk].long()].reshape(nblk * bs, 576)[:S, :512].float()
        lo.append(rows.amin(0))
        hi.append(rows.amax(0))
    lo = torch.stack(lo)[:, None, None]
    hi = torch.stack(hi)[:, None, None]
    slack = torch.maximum(lo.abs(), hi.abs()) * 2.0 ** -7 + 1e-6
    for label, f in launchers(case).items():
        print(f"mla_4k convex combination {label}", flush=True)
        out = f(case, False, SCALE)[0].float()
        assert torch.isfinite(out).all()
        below = (out < lo - slack).sum().item()
        above = (out > hi + slack).sum().item()
        assert below == 0 and above == 0, f"{label}: {below} below, {above} above"
