"""CPU tests that pin the oracle (oracle/reference.py and oracle/gqa_decode_oracle.c).

Every oracle function is checked against something it does not restate: the
reference's known-answer vectors (tests/golden/notes_w1_kat.json, from the
reference's docs/k1/notes_w1.md), torch's SDPA (the reference's own oracle
check, tests/test_reference.py:13-23), float64 brute force, closed forms, and
cases built so that a wrong head map, index or merge factor fails.
"""

import json
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import c_oracle
from oracle import reference as ref

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "notes_w1_kat.json")
D = 128


@pytest.fixture(scope="module")
def kat():
    with open(GOLDEN) as f:
        return json.load(f)


def random_bf16_case(rng, S_list, Hq, Hkv, bs, poison=True, std=1.0):
    """numpy mirror of the GPU case builder: bf16 bits, shuffled 2x pool,
    -1 padding, NaN in every slot that must not be read."""
    B = len(S_list)
    nb = [(s + bs - 1) // bs for s in S_list]
    pool = 2 * sum(nb)
    q = ref.f32_to_bf16(rng.standard_normal((B, Hq, D)).astype(np.float32) * std)
    k = ref.f32_to_bf16(rng.standard_normal((pool, bs, Hkv, D)).astype(np.float32) * std)
    v = ref.f32_to_bf16(rng.standard_normal((pool, bs, Hkv, D)).astype(np.float32) * std)
    perm = rng.permutation(pool)
    bt = np.full((B, max(nb)), -1, dtype=np.int32)
    used = np.zeros(pool, bool)
    off = 0
    for b in range(B):
        bt[b, :nb[b]] = perm[off:off + nb[b]]
        used[perm[off:off + nb[b]]] = True
        off += nb[b]
    if poison:
        nan = ref.f32_to_bf16(np.float32(np.nan))
        k[~used] = nan
        v[~used] = nan
        for b in range(B):
            if S_list[b] % bs:
                k[bt[b, nb[b] - 1], S_list[b] % bs:] = nan
                v[bt[b, nb[b] - 1], S_list[b] % bs:] = nan
    return q, k, v, bt, np.asarray(S_list, dtype=np.int32)


# ---------------------------------------------------------------- indexing


def test_kv_row_offset_kat(kat):
    k = kat["paged_index"]
    bt = np.asarray(k["block_table"], dtype=np.int32)
    off = ref.kv_row_offset(bt, k["token"], k["block_size"], k["Hkv"], k["head"])
    assert off == k["element_offset"]
    assert off * 2 == k["byte_offset"]
    assert c_oracle.kv_offset(bt, k["token"], k["block_size"], k["Hkv"], k["head"]) == off


def test_gather_kv_reads_only_live_slots():
    # Values encode (block, slot, head, dim); dead slots are NaN.
    pool, bs, Hkv = 6, 4, 2
    kc = np.full((pool, bs, Hkv, D), np.nan, dtype=np.float32)
    p, s, h, d = np.meshgrid(np.arange(pool), np.arange(bs), np.arange(Hkv), np.arange(D),
                             indexing="ij")
    code = ((p * 1000 + s * 100 + h * 10) + d / 1000.0).astype(np.float32)
    bt = np.array([[4, 1, 3, -1]], dtype=np.int32)
    S = 10  # blocks 4, 1 full; block 3 holds two live slots
    live = np.zeros_like(kc, dtype=bool)
    live[4] = live[1] = True
    live[3, :2] = True
    kc[live] = code[live]
    K, V = ref.gather_kv(kc, kc.copy(), bt, S, 0)
    assert K.shape == (S, Hkv, D) and np.isfinite(K).all()
    for t in range(S):
        blk, slot = bt[0, t // bs], t % bs
        np.testing.assert_array_equal(K[t], code[blk, slot])


# ------------------------------------------------------------ attention_ref


def sdpa_check(B, S, Hq, Hkv):
    """Oracle vs F.scaled_dot_product_attention on fp32 data, identity table
    (the reference's check_against_sdpa, python/reference.py:43-75)."""
    rng = np.random.default_rng(0)
    bs = 16
    mb = (max(S) + bs - 1) // bs
    nblk = B * mb
    q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    k = rng.standard_normal((nblk, bs, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((nblk, bs, Hkv, D)).astype(np.float32)
    bt = np.arange(nblk, dtype=np.int32).reshape(B, mb)
    scale = 1.0 / math.sqrt(D)
    out = ref.attention_ref(q, k, v, bt, np.asarray(S), scale)
    err = 0.0
    for b in range(B):
        K, V = ref.gather_kv(k, v, bt, S[b], b)
        Ke = torch.from_numpy(K).permute(1, 0, 2).repeat_interleave(Hq // Hkv, dim=0)
        Ve = torch.from_numpy(V).permute(1, 0, 2).repeat_interleave(Hq // Hkv, dim=0)
        o = F.scaled_dot_product_attention(torch.from_numpy(q[b]).unsqueeze(1), Ke, Ve,
                                           scale=scale)
        err = max(err, float((o.squeeze(1).numpy() - out[b]).__abs__().max()))
    return err


@pytest.mark.parametrize("B,S,Hq,Hkv", [(2, [37, 100], 32, 8), (1, [1], 32, 8),
                                        (3, [16, 17, 64], 64, 8)])
def test_attention_ref_matches_sdpa(B, S, Hq, Hkv):
    assert sdpa_check(B, S, Hq, Hkv) < 1e-5


def brute_force(q, k, v, bt, S_list, scale):
    """float64 pure-Python evaluation of the definition (tiny inputs only)."""
    B, Hq, _ = q.shape
    _, bs, Hkv, _ = k.shape
    out = np.zeros((B, Hq, D))
    for b in range(B):
        for h in range(Hq):
            kv = h // (Hq // Hkv)
            rows = [(bt[b][t // bs], t % bs) for t in range(S_list[b])]
            s = [scale * sum(float(q[b, h, d]) * float(k[p, sl, kv, d]) for d in range(D))
                 for p, sl in rows]
            mx = max(s)
            w = [math.exp(x - mx) for x in s]
            tot = sum(w)
            for d in range(D):
                out[b, h, d] = sum(w[i] * float(v[p, sl, kv, d])
                                   for i, (p, sl) in enumerate(rows)) / tot
    return out


def test_attention_ref_brute_force():
    rng = np.random.default_rng(1)
    S_list = [3, 5]
    q, k, v, bt, sl = random_bf16_case(rng, S_list, Hq=4, Hkv=2, bs=2)
    scale = 1.0 / math.sqrt(D)
    got = ref.attention_ref(q, k, v, bt, sl, scale)
    want = brute_force(ref.bf16_to_f32(q), ref.bf16_to_f32(k), ref.bf16_to_f32(v), bt, S_list,
                       scale)
    np.testing.assert_allclose(got, want, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(c_oracle.attention_ref(q, k, v, bt, sl, scale), want, atol=1e-5,
                               rtol=1e-5)


def test_closed_forms():
    rng = np.random.default_rng(2)
    scale = 1.0 / math.sqrt(D)
    # S = 1: the softmax weight is 1, so out = V[0] exactly.
    q, k, v, bt, sl = random_bf16_case(rng, [1, 1], Hq=8, Hkv=2, bs=16)
    for impl in (ref.attention_ref, c_oracle.attention_ref):
        out = impl(q, k, v, bt, sl, scale)
        for b in range(2):
            for h in range(8):
                np.testing.assert_array_equal(out[b, h], ref.bf16_to_f32(v[bt[b, 0], 0, h // 4]))
    # Identical keys: uniform weights, out = mean of the V rows.
    q, k, v, bt, sl = random_bf16_case(rng, [37], Hq=4, Hkv=1, bs=8, poison=False)
    k[:] = k[bt[0, 0], 0]
    K, V = ref.gather_kv(k, v, bt, 37, 0)
    for impl in (ref.attention_ref, c_oracle.attention_ref):
        out = impl(q, k, v, bt, sl, scale)
        np.testing.assert_allclose(out[0], np.broadcast_to(V[:, 0].mean(0), (4, D)), atol=1e-6)
    # One dominant key: out = its V row.
    q, k, v, bt, sl = random_bf16_case(rng, [50], Hq=1, Hkv=1, bs=16, poison=False)
    qf = ref.bf16_to_f32(q[0, 0])
    t_star = 23
    k[bt[0, t_star // 16], t_star % 16, 0] = ref.f32_to_bf16(qf * 8.0)
    out = ref.attention_ref(q, k, v, bt, sl, 1.0)
    np.testing.assert_allclose(out[0, 0], ref.bf16_to_f32(v[bt[0, 1], 7, 0]), atol=1e-6)


def test_head_map_is_consecutive_grouping():
    """V rows of kv-head j are all equal to j, so out[b, h] = h // G; the
    strided rule kv = h % Hkv (docs/decisions/k1-002) would give h % Hkv."""
    rng = np.random.default_rng(3)
    Hq, Hkv = 16, 4
    q, k, v, bt, sl = random_bf16_case(rng, [20, 9], Hq=Hq, Hkv=Hkv, bs=4, poison=False)
    for j in range(Hkv):
        v[:, :, j, :] = ref.f32_to_bf16(np.float32(j))
    for impl in (ref.attention_ref, c_oracle.attention_ref):
        out = impl(q, k, v, bt, sl, 0.1)
        for h in range(Hq):
            np.testing.assert_allclose(out[:, h], h // (Hq // Hkv), atol=1e-6)


def test_online_softmax_kat(kat):
    """Scores [2,5,1,6] with 2-d values (notes_w1.md:74-86): q = e0, K[t,0] = s_t,
    scale 1 make the scores exact."""
    t = kat["online_softmax"]
    S = len(t["scores"])
    q = np.zeros((1, 1, D), np.float32)
    q[0, 0, 0] = 1.0
    k = np.zeros((1, S, 1, D), np.float32)
    v = np.zeros((1, S, 1, D), np.float32)
    k[0, :, 0, 0] = t["scores"]
    v[0, :, 0, :2] = t["values"]
    bt = np.zeros((1, 1), np.int32)
    out = ref.attention_ref(q, k, v, bt, [S], 1.0)
    np.testing.assert_allclose(out[0, 0, :2], t["out"], atol=1e-4)
    for i, step in enumerate(t["trace"]):
        m, l, acc = ref.partial_state(q[0, 0], k[0, :i + 1, 0], v[0, :i + 1, 0], 1.0)
        assert m == step["m"]
        assert l == pytest.approx(step["l"], abs=1e-6)
        np.testing.assert_allclose(acc[:2], step["acc"], atol=1e-6)
    qb = ref.f32_to_bf16(q)
    kb, vb = ref.f32_to_bf16(k), ref.f32_to_bf16(v)
    np.testing.assert_allclose(c_oracle.attention_ref(qb, kb, vb, bt, [S], 1.0)[0, 0, :2],
                               t["out"], atol=1e-4)


def test_split_merge_kat(kat):
    t = kat["split_merge"]
    o = kat["online_softmax"]
    q = np.zeros(D)
    q[0] = 1.0
    K = np.zeros((4, D))
    V = np.zeros((4, D))
    K[:, 0] = o["scores"]
    V[:, :2] = o["values"]
    states = []
    for key in ("split1", "split2"):
        sp = t[key]
        m, l, acc = ref.partial_state(q, K[sp["tokens"]], V[sp["tokens"]], 1.0)
        assert m == sp["m"] and l == pytest.approx(sp["l"], abs=1e-6)
        np.testing.assert_allclose(acc[:2], sp["acc"], atol=1e-6)
        states.append((m, l, acc))
    ms, ls, accs = zip(*states)
    for merge in (lambda: ref.merge_states(ms, ls, np.stack(accs))[0],
                  lambda: c_oracle.merge_states(ms, ls, np.stack(accs))):
        np.testing.assert_allclose(merge()[:2], t["merged"]["out"], atol=1e-4)
    _, _, L = ref.merge_states(ms, ls, np.stack(accs))
    assert L == pytest.approx(t["merged"]["l"], abs=1e-6)


@pytest.mark.parametrize("ns", [1, 3, 8, 32])
def test_split_merge_equals_attention(ns):
    """Any segmentation (reference rule, empty segments included) merges back to
    the single-pass result; the C restatement of both steps agrees."""
    rng = np.random.default_rng(4)
    S_list = [100, 1, 33]
    q, k, v, bt, sl = random_bf16_case(rng, S_list, Hq=8, Hkv=2, bs=16)
    scale = 1.0 / math.sqrt(D)
    want = ref.attention_ref(q, k, v, bt, sl, scale)
    for b, S in enumerate(S_list):
        K, V = ref.gather_kv(k, v, bt, S, b)
        for h in range(8):
            kv = h // 4
            segs = ref.split_bounds(S, ns)
            st = [ref.partial_state(ref.bf16_to_f32(q[b, h]), K[a:e, kv], V[a:e, kv], scale)
                  for a, e in segs]
            ms, ls, accs = zip(*st)
            got, _, _ = ref.merge_states(ms, ls, np.stack(accs))
            np.testing.assert_allclose(got, want[b, h], atol=2e-6, rtol=1e-5)
            cst = [c_oracle.partial_state(q[b, h], k, v, bt[b], kv, a, e, scale)
                   for a, e in segs]
            for (m1, l1, a1), (m2, l2, a2) in zip(st, cst):
                assert m1 == pytest.approx(m2, abs=1e-6) and l1 == pytest.approx(l2, rel=1e-6)
                np.testing.assert_allclose(a1, a2, atol=1e-5)
            cm, cl, ca = zip(*cst)
            np.testing.assert_allclose(c_oracle.merge_states(cm, cl, np.stack(ca)), want[b, h],
                                       atol=2e-6, rtol=1e-5)


def test_split_bounds_reference_rule():
    assert ref.split_bounds(100, 8) == [(0, 13), (13, 26), (26, 39), (39, 52), (52, 65),
                                       (65, 78), (78, 91), (91, 100)]
    assert ref.split_bounds(1, 8) == [(0, 1)] + [(1, 1)] * 7


def test_empty_segment_state():
    m, l, acc = ref.partial_state(np.ones(D), np.zeros((0, D)), np.zeros((0, D)), 1.0)
    assert m == -math.inf and l == 0.0 and not acc.any()


def test_c_oracle_matches_numpy_oracle():
    rng = np.random.default_rng(5)
    q, k, v, bt, sl = random_bf16_case(rng, [300, 17, 1, 64, 257], Hq=32, Hkv=8, bs=16)
    scale = 1.0 / math.sqrt(D)
    a = ref.attention_ref(q, k, v, bt, sl, scale)
    b = c_oracle.attention_ref(q, k, v, bt, sl, scale, nthreads=4)
    assert np.isfinite(a).all()
    np.testing.assert_allclose(a, b, atol=2e-6, rtol=1e-5)


def test_f32_to_bf16_round_to_nearest_even():
    rng = np.random.default_rng(6)
    x = np.concatenate([
        rng.standard_normal(10000).astype(np.float32) * 10,
        # exact ties between two bf16 values, both parities
        (np.arange(1, 2000, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38, 1e-40], dtype=np.float32),
    ])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ref.f32_to_bf16(x), want)
    assert np.isnan(ref.bf16_to_f32(ref.f32_to_bf16(np.float32(np.nan))))
    np.testing.assert_array_equal(ref.bf16_to_f32(want), torch.from_numpy(x).to(
        torch.bfloat16).float().numpy())
