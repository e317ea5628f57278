"""GPU checks of exact properties of the attention at the five BASELINE.json
configs' full sizes, with no oracle in the loop.

Decode attention is out[b, h] = sum_t w_t V[t, kv(h)] with weights
w = softmax(scale * <q[b, h], K[t, kv(h)]>) over the request's tokens. On
the same inputs:
- V enters linearly: doubling V doubles every product, sum and state of every
  scan and merge exactly (binary floating point scales by 2 without rounding),
  so out(q, K, 2V) == 2 out(q, K, V) bit for bit;
- K enters only through the scaled dot product: out(q, 2K, V, scale / 2) ==
  out(q, K, V, scale) bit for bit;
- out is a convex combination of its kv-head's V rows: every element lies
  between the smallest and largest value of its dimension over the request's
  tokens (up to the bf16 rounding of out);
- attending to every token twice leaves the weights unchanged: a block table
  that lists each request's blocks twice, with twice the length, gives the
  same output within the bf16 tolerance.
A kernel that swapped K and V, dropped the 1/l normalisation, misplaced the
scale or mishandled a block id that repeats fails one of these, at the sizes
the bench runs. Each case prints what it runs before it runs it.
"""

import math

import pytest
import torch

from binding import gqa_decode_v0, gqa_decode_v1, gqa_decode_v2
from cases import CONFIGS, make_config_case
from gpu_util import assert_close

pytestmark = pytest.mark.gpu

SCALE = 1.0 / math.sqrt(128)
TOL = 1e-2

LAUNCHES = {
    "v1": lambda *a: gqa_decode_v1(*a),
    "v2/4": lambda *a: gqa_decode_v2(*a, num_splits=4),
    "v2/32": lambda *a: gqa_decode_v2(*a, num_splits=32),
    "v2/auto": lambda *a: gqa_decode_v2(*a, num_splits=0),
}


@pytest.fixture(scope="module")
def cases():
    store = {}

    def get(name):  # all five stay resident (~16 GiB): each test walks them in turn
        if name not in store:
            print(f"building config {name}", flush=True)
            store[name] = make_config_case(name, seed=3, poison=(name == "c5"))
        return store[name]
    yield get
    store.clear()
    torch.cuda.empty_cache()


def launches(name):
    out = dict(LAUNCHES)
    if name == "c1":
        out["v0"] = lambda *a: gqa_decode_v0(*a)
    return out


@pytest.mark.parametrize("name", list(CONFIGS))
def test_v_linearity(gpu, cases, name):
    q, k, v, bt, sl = cases(name)
    v2 = v * 2  # exact in bf16 (|v| far below the overflow bound); NaN stays NaN
    for label, fn in launches(name).items():
        print(f"{name} V linearity {label}", flush=True)
        want = fn(q, k, v, bt, sl, SCALE) * 2
        got = fn(q, k, v2, bt, sl, SCALE)
        assert torch.equal(got, want), f"{name}/{label}: out(2V) != 2 out(V)"
    del v2
    torch.cuda.empty_cache()


@pytest.mark.parametrize("name", list(CONFIGS))
def test_k_scale(gpu, cases, name):
    q, k, v, bt, sl = cases(name)
    k2 = k * 2
    for label, fn in launches(name).items():
        print(f"{name} K scale {label}", flush=True)
        want = fn(q, k, v, bt, sl, SCALE)
        got = fn(q, k2, v, bt, sl, SCALE / 2)
        assert torch.equal(got, want), f"{name}/{label}: out(2K, scale/2) != out(K, scale)"
    del k2
    torch.cuda.empty_cache()


def value_bounds(case):
    """Per (request, kv-head, dim): min and max of V over the request's tokens."""
    q, k, v, bt, sl = case
    bs = v.shape[1]
    lo, hi = [], []
    for b, S in enumerate(sl.tolist()):
        nblk = -(-S // bs)
        rows = v[bt[b, :nblk].long()].reshape(nblk * bs, v.shape[2], v.shape[3])[:S].float()
        lo.append(rows.amin(0))
        hi.append(rows.amax(0))
    return torch.stack(lo), torch.stack(hi)


@pytest.mark.parametrize("name", list(CONFIGS))
def test_convex_combination(gpu, cases, name):
    case = cases(name)
    q, k = case[0], case[1]
    G = q.shape[1] // k.shape[2]
    lo, hi = value_bounds(case)
    lo = lo.repeat_interleave(G, dim=1)  # kv-head of q-head h: h // G
    hi = hi.repeat_interleave(G, dim=1)
    slack = torch.maximum(lo.abs(), hi.abs()) * 2.0 ** -7 + 1e-6  # two bf16 ulps
    for label, fn in launches(name).items():
        print(f"{name} convex combination {label}", flush=True)
        out = fn(*case, SCALE).float()
        assert torch.isfinite(out).all(), f"{name}/{label}"
        below = (out < lo - slack).sum().item()
        above = (out > hi + slack).sum().item()
        assert below == 0 and above == 0, f"{name}/{label}: {below} below, {above} above"


@pytest.mark.parametrize("name", ["c2", "c3", "c4"])
def test_every_token_twice(gpu, cases, name):
    q, k, v, bt, sl = cases(name)
    assert all(s % k.shape[1] == 0 for s in sl.tolist())  # whole blocks: the copy aligns
    twice = (q, k, v, torch.cat([bt, bt], dim=1).contiguous(), (sl * 2).contiguous())
    for label, fn in LAUNCHES.items():
        print(f"{name} every token twice {label}", flush=True)
        want = fn(q, k, v, bt, sl, SCALE).float().cpu().numpy()
        got = fn(*twice, SCALE).float().cpu().numpy()
        assert_close(got, want, TOL, TOL, f"{name}/{label} twice")
