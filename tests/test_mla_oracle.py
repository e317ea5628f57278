"""CPU tests that pin the MLA decode oracle (oracle/mla_reference.py and its C
restatement oracle/mla_decode_oracle.c).

The reference has no MLA implementation or golden vectors (its
kernels/mla_decode/ is empty; README.md:405-408 of the reference names the
item and FlashMLA at 15f13e5 as its baseline). The oracle restates FlashMLA's
published decode semantics, and these checks fix what the mathematics fixes:
  - closed forms: one token -> its value row and lse = its score; q = 0 ->
    the mean of the value rows and lse = log S; one key far above the rest ->
    that key's value row;
  - float64 brute force with explicit loops on tiny inputs;
  - an independent torch float32 computation (scaled_dot_product_attention
    with an explicit boolean mask, and torch.logsumexp);
  - the paged gather against a contiguous cache holding the same rows;
  - the causal mask against per-query truncation of the sequence;
  - the C restatement against the numpy one;
  - a mistake planted in a copy of the oracle (value rows taken from the
    wrong 512 dims) is caught.
"""

import math

import numpy as np
import pytest
import torch

from cases import make_mla_case, mla_flops_bytes
from oracle import c_oracle
from oracle import mla_reference as mref
from oracle.reference import bf16_to_f32

SCALE = 576 ** -0.5


def host(case):
    q, kv, bt, sl = case
    bits = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)
    return bits(q), bits(kv), bt.numpy(), sl.numpy()


def rows_of(kv, bt_row, S):
    """Request rows by explicit per-token indexing (independent of the
    oracle's gather): [S, 576] float64."""
    bs = kv.shape[1]
    return np.stack([bf16_to_f32(kv[bt_row[t // bs], t % bs, 0]) for t in range(S)]).astype(
        np.float64)


def case(S_list, s_q=1, h_q=4, bs=16, seed=0, poison=True, shuffle=True):
    return host(make_mla_case(S_list, s_q, h_q, bs, pool_factor=2, seed=seed, device="cpu",
                              poison=poison, shuffle=shuffle))


def test_one_token_is_its_value_row():
    q, kv, bt, sl = case([1], s_q=1, h_q=3)
    out, lse = mref.mla_decode_ref(q, kv, bt, sl, SCALE)
    row = bf16_to_f32(kv[bt[0, 0], 0, 0])
    np.testing.assert_array_equal(out[0, 0], np.broadcast_to(row[:512], (3, 512)))
    want = SCALE * (bf16_to_f32(q[0, 0]).astype(np.float64) @ row.astype(np.float64))
    np.testing.assert_allclose(lse[0, :, 0], want, rtol=1e-6)


def test_zero_query_is_the_mean_and_log_length():
    q, kv, bt, sl = case([37], h_q=2)
    q[:] = 0
    out, lse = mref.mla_decode_ref(q, kv, bt, sl, SCALE)
    rows = rows_of(kv, bt[0], 37)
    np.testing.assert_allclose(out[0, 0, 0], rows[:, :512].mean(axis=0), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(lse[0, :, 0], math.log(37), rtol=1e-7)


def test_dominant_key_selects_its_row():
    q, kv, bt, sl = case([50], h_q=1, poison=False)
    rows = rows_of(kv, bt[0], 50).astype(np.float32)
    # Query = 64 x key 17: its score beats every other by far more than e^30.
    target = rows[17]
    qv = torch.from_numpy(target * 64.0).to(torch.bfloat16).view(torch.int16).numpy()
    q[0, 0, 0] = qv.view(np.uint16)
    out, _ = mref.mla_decode_ref(q, kv, bt, sl, 1.0)
    np.testing.assert_allclose(out[0, 0, 0], target[:512], rtol=1e-5, atol=1e-6)


def brute_force(q, kv, bt, sl, scale, causal):
    B, s_q, h_q, _ = q.shape
    bs = kv.shape[1]
    out = np.zeros((B, s_q, h_q, 512))
    lse = np.full((B, h_q, s_q), -np.inf)
    for b in range(B):
        for i in range(s_q):
            lim = int(sl[b]) - (s_q - 1 - i) if causal else int(sl[b])
            for h in range(h_q):
                qv = [float(x) for x in bf16_to_f32(q[b, i, h])]
                scores, vals = [], []
                for t in range(max(lim, 0)):
                    c = bf16_to_f32(kv[bt[b, t // bs], t % bs, 0])
                    scores.append(scale * sum(qv[d] * float(c[d]) for d in range(576)))
                    vals.append(c[:512].astype(np.float64))
                if not scores:
                    continue
                m = max(scores)
                w = [math.exp(x - m) for x in scores]
                tot = sum(w)
                out[b, i, h] = sum(wi * v for wi, v in zip(w, vals)) / tot
                lse[b, h, i] = m + math.log(tot)
    return out, lse


@pytest.mark.parametrize("causal", [False, True])
def test_brute_force(causal):
    q, kv, bt, sl = case([5, 3, 1], s_q=2, h_q=2, bs=4, seed=3)
    out, lse = mref.mla_decode_ref(q, kv, bt, sl, SCALE, causal=causal)
    want_out, want_lse = brute_force(q, kv, bt, sl, SCALE, causal)
    np.testing.assert_allclose(out, want_out, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(lse, want_lse, rtol=1e-6)


@pytest.mark.parametrize("causal", [False, True])
def test_against_torch_sdpa(causal):
    S_list = [70, 1, 33, 128]
    s_q, h_q = 2, 8
    q, kv, bt, sl = case(S_list, s_q=s_q, h_q=h_q, bs=16, seed=4)
    out, lse = mref.mla_decode_ref(q, kv, bt, sl, SCALE, causal=causal)
    for b, S in enumerate(S_list):
        C = torch.from_numpy(rows_of(kv, bt[b], S).astype(np.float32))   # [S, 576]
        Q = torch.from_numpy(bf16_to_f32(q[b])).reshape(s_q * h_q, 576)   # rows (i, h)
        qi = torch.arange(s_q).repeat_interleave(h_q)
        lim = torch.full_like(qi, S) - ((s_q - 1 - qi) if causal else 0)
        mask = torch.arange(S)[None, :] < lim[:, None]
        got = torch.nn.functional.scaled_dot_product_attention(
            Q[None], C[None], C[None, :, :512], attn_mask=mask[None], scale=SCALE)[0]
        live = lim > 0
        np.testing.assert_allclose(out[b].reshape(s_q * h_q, 512)[live.numpy()],
                                   got[live].numpy(), rtol=1e-4, atol=1e-5)
        scores = (Q @ C.T) * SCALE
        ref_lse = torch.logsumexp(scores.masked_fill(~mask, -math.inf), dim=1)
        np.testing.assert_allclose(lse[b].T.reshape(-1)[live.numpy()],
                                   ref_lse[live].numpy(), rtol=1e-5, atol=1e-5)


def test_paged_equals_contiguous():
    # The same rows under shuffled block ids and in a contiguous cache with an
    # identity table give the same bits.
    S_list = [100, 17, 64]
    q, kv, bt, sl = case(S_list, h_q=3, bs=16, seed=5, poison=True, shuffle=True)
    got = mref.mla_decode_ref(q, kv, bt, sl, SCALE)
    for b, S in enumerate(S_list):
        nblk = -(-S // 16)
        contig = np.stack([kv[bt[b, k]] for k in range(nblk)])       # [nblk, 16, 1, 576]
        ident = np.arange(nblk, dtype=np.int32)[None]
        want = mref.mla_decode_ref(q[b:b + 1], contig, ident, sl[b:b + 1], SCALE)
        np.testing.assert_array_equal(got[0][b], want[0][0])
        np.testing.assert_array_equal(got[1][b], want[1][0])


def test_causal_is_truncation():
    q, kv, bt, sl = case([40], s_q=3, h_q=2, bs=16, seed=6)
    out, lse = mref.mla_decode_ref(q, kv, bt, sl, SCALE, causal=True)
    for i in range(3):
        lim = 40 - (2 - i)
        o_i, l_i = mref.mla_decode_ref(q[:, i:i + 1], kv, bt, np.array([lim], np.int32), SCALE)
        np.testing.assert_array_equal(out[0, i], o_i[0, 0])
        np.testing.assert_array_equal(lse[0, :, i], l_i[0, :, 0])


def test_empty_rows():
    q, kv, bt, sl = case([0, 2], s_q=3, h_q=2, bs=16, seed=7)
    out, lse = mref.mla_decode_ref(q, kv, bt, sl, SCALE, causal=True)
    assert not out[0].any() and np.isneginf(lse[0]).all()
    # Request 1 (2 tokens, 3 query tokens, causal): query 0 sees none.
    assert not out[1, 0].any() and np.isneginf(lse[1, :, 0]).all()
    assert np.isfinite(lse[1, :, 1:]).all()


@pytest.mark.parametrize("causal", [False, True])
def test_c_oracle_matches_numpy(causal):
    q, kv, bt, sl = case([300, 1, 65, 0, 129], s_q=2, h_q=5, bs=64, seed=8)
    want = mref.mla_decode_ref(q, kv, bt, sl, SCALE, causal=causal)
    got = c_oracle.mla_decode_ref(q, kv, bt, sl, SCALE, causal=causal)
    np.testing.assert_allclose(got[0], want[0], rtol=1e-6, atol=1e-7)
    np.testing.assert_array_equal(np.isneginf(got[1]), np.isneginf(want[1]))
    fin = np.isfinite(want[1])
    np.testing.assert_allclose(got[1][fin], want[1][fin], rtol=1e-6)


def test_planted_mistake_is_caught(monkeypatch):
    # Values taken from dims 64..576 instead of 0..512: the closed forms and the
    # torch comparison must fail.
    real = mref.gather_latent

    def wrong(kv, bt_row, S):
        rows = real(kv, bt_row, S)
        return np.concatenate([rows[:, 64:], rows[:, :64]], axis=1)

    monkeypatch.setattr(mref, "gather_latent", wrong)
    for pin in (test_zero_query_is_the_mean_and_log_length, test_one_token_is_its_value_row,
                lambda: test_against_torch_sdpa(False)):
        with pytest.raises(AssertionError):
            pin()


def test_flops_bytes_accounting():
    # The benchmark's accounting (bench/cases.py), FlashMLA's counting for b=128, s_q=1, h_q=128, every request at 32768:
    # 128*128*32768*2*(576+512) FLOPs; bytes = q + latent rows once + out.
    flops, nbytes = mla_flops_bytes([32768] * 128, 1, 128)
    assert flops == 2.0 * 128 * 128 * 32768 * 1088
    assert nbytes == 128 * 128 * 576 * 2 + 128 * 32768 * 576 * 2 + 128 * 128 * 512 * 2


@pytest.mark.parametrize("s_q,s_k,tflops,gbps", [
    (1, 4096, 535, 2344), (1, 8192, 583, 2480), (1, 16384, 610, 2561), (1, 32768, 627, 2612),
    (2, 4096, 690, 1595), (2, 8192, 729, 1597), (2, 16384, 751, 1598), (2, 32768, 758, 1592)])
def test_accounting_matches_flashmla_log(s_q, s_k, tflops, gbps):
    # FlashMLA's printed rows (docs/g0/flashmla_bench_raw.txt:4675-4697 of the
    # reference) fix the ratio of its byte count to its FLOP count, whatever
    # the varlen draw's total: both counts must be the ones it used.
    flops, nbytes = mla_flops_bytes([s_k] * 128, s_q, 128)
    assert abs((nbytes / flops) / (gbps / (tflops * 1e3)) - 1) < 0.01
