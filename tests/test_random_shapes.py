"""GPU parity over seeded random shapes, against the C oracle.

The launch a shape takes depends on the group size, kv-head count, batch,
block size, longest length, split count and the device's CU count: the VALU
or matrix-core scan, the shared or split-range layout, 4 to 16 waves per
split on grids that leave CUs idle, the matrix-core scan for short splits
there, the slot-group layout, the token-balanced launch under the automatic
choice. 30 seeded shapes (kv-heads 1-16, groups 1-8, up to 16 ragged
requests of up to 4096 tokens, block sizes on and off the 16-token tile,
NaN in every slot that must not be read) run v1, v2 at a random split
count and at the automatic choice; every output is checked against the
oracle (atol = rtol = 1e-2) and v2 with one split against v1, bit for bit.
Each shape prints its parameters before it runs.
"""

import math

import numpy as np
import pytest
import torch

from binding import gqa_decode_v1, gqa_decode_v2
from cases import make_case
from gpu_util import assert_close, oracle

pytestmark = pytest.mark.gpu

SCALE = 1.0 / math.sqrt(128)
TOL = 1e-2


def shapes(n=30, seed=77):
    rng = np.random.default_rng(seed)
    for i in range(n):
        Hkv = int(rng.choice([1, 2, 4, 8, 16]))
        G = int(rng.integers(1, 9))
        B = int(rng.integers(1, 17))
        bs = int(rng.choice([1, 7, 16, 64]))
        top = int(rng.choice([64, 1024, 4096]))
        S = rng.integers(1, top + 1, size=B).tolist()
        ns = int(rng.choice([2, 3, 4, 8, 16, 32, 64]))
        yield i, Hkv, G, B, bs, S, ns


@pytest.mark.parametrize("i,Hkv,G,B,bs,S,ns", list(shapes()))
def test_random_shape(gpu, i, Hkv, G, B, bs, S, ns):
    print(f"shape {i}: Hq={G * Hkv} Hkv={Hkv} B={B} bs={bs} max S={max(S)} ns={ns}", flush=True)
    case = make_case(S, G * Hkv, Hkv, bs, pool_factor=1.25, seed=i, qkv_std=0.5, poison=True)
    want = oracle(case, SCALE)
    out1 = gqa_decode_v1(*case, SCALE)
    for label, fn in (("v1", lambda: out1),
                      ("v2/1", lambda: gqa_decode_v2(*case, SCALE, num_splits=1)),
                      (f"v2/{ns}", lambda: gqa_decode_v2(*case, SCALE, num_splits=ns)),
                      ("v2/auto", lambda: gqa_decode_v2(*case, SCALE, num_splits=0))):
        out = fn()
        torch.cuda.synchronize()
        assert_close(out, want, TOL, TOL, f"shape {i} {label}")
        if label == "v2/1":
            assert torch.equal(out, out1), f"shape {i}: v2 with one split != v1"
