"""GPU parity on the five BASELINE.json configs at their full sizes.

Inputs are N(0,1) bf16 from a stated seed, compared
to the fp32 oracle with atol = rtol = 1e-2 (north_star). C1-C3 are checked on
every request; C4 (4 GiB) and C5 (ragged, ~10 GiB pool) on a request subset
that includes the shortest and longest requests, plus size-independent
properties on the whole batch: v2(ns=1) == v1 bitwise, bitwise repeatability,
and agreement between split counts.
"""

import math

import numpy as np
import pytest
import torch

from binding import gqa_decode_v0, gqa_decode_v1, gqa_decode_v2
from cases import CONFIGS, config_seq_lens, make_config_case
from gpu_util import assert_close, oracle

pytestmark = pytest.mark.gpu

TOL = 1e-2
SCALE = 1.0 / math.sqrt(128)


@pytest.fixture(scope="module")
def cases():
    store = {}

    def get(name):
        if name not in store:
            store.clear()
            torch.cuda.empty_cache()
            print(f"building config {name}", flush=True)
            store[name] = make_config_case(name, seed=0, poison=(name == "c5"))
        return store[name]
    return get


def check_subset(out, case, batches, label):
    want = oracle(case, SCALE, batches)
    assert_close(out[batches], want, TOL, TOL, label)


SPLITS = {"c1": [1, 4, 8, 16, 32], "c2": [1, 4, 8, 16, 32], "c3": [1, 4, 8, 16, 32, 64],
          "c4": [0], "c5": [0]}


def subset(name):
    B = CONFIGS[name]["B"]
    if name in ("c1", "c2", "c3"):
        return list(range(B))
    S = config_seq_lens(name)
    order = np.argsort(S)
    return sorted(set([int(order[0]), int(order[-1]), 0, B - 1, B // 2, B // 3]))


@pytest.mark.parametrize("name", list(CONFIGS))
def test_config_v2(gpu, cases, name):
    case = cases(name)
    batches = subset(name)
    want = oracle(case, SCALE, batches)
    outs = {}
    for ns in SPLITS[name] + [0]:
        print(f"{name} v2 num_splits={ns}", flush=True)
        out = gqa_decode_v2(*case, SCALE, num_splits=ns)
        torch.cuda.synchronize()
        assert torch.isfinite(out.float()).all()
        assert_close(out[batches], want, TOL, TOL, f"{name}/v2/ns{ns}")
        outs[ns] = out
    # Different split counts agree on every request, not only the checked subset.
    base = outs[0].float()
    for ns, out in outs.items():
        assert_close(out.float().cpu().numpy(), base.cpu().numpy(), TOL, TOL, f"{name} ns{ns}~h")


@pytest.mark.parametrize("name", list(CONFIGS))
def test_config_v1_and_identity(gpu, cases, name):
    case = cases(name)
    print(f"{name} v1", flush=True)
    out1 = gqa_decode_v1(*case, SCALE)
    torch.cuda.synchronize()
    check_subset(out1, case, subset(name), f"{name}/v1")
    assert torch.equal(gqa_decode_v2(*case, SCALE, num_splits=1), out1)
    assert torch.equal(gqa_decode_v1(*case, SCALE), out1)
    outh = gqa_decode_v2(*case, SCALE, num_splits=0)
    for _ in range(3):
        assert torch.equal(gqa_decode_v2(*case, SCALE, num_splits=0), outh)


@pytest.mark.parametrize("name", ["c1", "c2"])
def test_config_v0(gpu, cases, name):
    case = cases(name)
    out = gqa_decode_v0(*case, SCALE)
    torch.cuda.synchronize()
    check_subset(out, case, subset(name), f"{name}/v0")


def move_blocks(case, seed):
    """The same logical cache with every physical block moved to a new slot
    of the pool (block table remapped; padding entries stay -1)."""
    q, k, v, bt, sl = case
    perm = torch.randperm(k.shape[0], generator=torch.Generator().manual_seed(seed)).to(k.device)
    k2, v2 = torch.empty_like(k), torch.empty_like(v)
    k2[perm] = k
    v2[perm] = v
    bt2 = torch.where(bt >= 0, perm[bt.clamp_min(0).long()].to(torch.int32), bt)
    return q, k2, v2, bt2, sl


LAUNCHES = {
    "v1": lambda *a: gqa_decode_v1(*a),
    "v2/4": lambda *a: gqa_decode_v2(*a, num_splits=4),
    "v2/auto": lambda *a: gqa_decode_v2(*a, num_splits=0),
}


@pytest.mark.parametrize("name", ["c2", "c4", "c5"])
def test_config_layout_invariance(gpu, cases, name):
    # Where the blocks sit in the pool changes only addresses: every launch
    # reads the same values in the same order, so the output is bitwise equal.
    case = cases(name)
    moved = move_blocks(case, seed=1)
    for label, fn in LAUNCHES.items():
        print(f"{name} layout {label}", flush=True)
        assert torch.equal(fn(*case, SCALE), fn(*moved, SCALE)), f"{name}/{label}"
    del moved
    torch.cuda.empty_cache()


@pytest.mark.parametrize("name", ["c3", "c5"])
def test_config_request_order(gpu, cases, name):
    # Permuting the batch permutes the output rows: bitwise for the split
    # launches (requests are independent); the automatic choice may run the
    # token-balanced launch, whose shares move with the order: within 1e-2.
    q, k, v, bt, sl = cases(name)
    p = torch.randperm(q.shape[0], generator=torch.Generator().manual_seed(2)).to(q.device)
    shuffled = (q[p].contiguous(), k, v, bt[p].contiguous(), sl[p].contiguous())
    for label, fn in LAUNCHES.items():
        print(f"{name} request order {label}", flush=True)
        want = fn(q, k, v, bt, sl, SCALE)[p]
        got = fn(*shuffled, SCALE)
        if label == "v2/auto":
            assert_close(got.float().cpu().numpy(), want.float().cpu().numpy(), TOL, TOL, label)
        else:
            assert torch.equal(got, want), f"{name}/{label}"
