"""GPU parity at the edges of the shape space the C ABI accepts.

The reference's grid (tests/test_gqa_decode.py:89-98 of the reference) stays
within 32-64 q-heads, 8 kv-heads, blocks of 16/64 and sequences of 8192.
These cases push each dimension further, against the fp32 oracle with the
reference's inputs and tolerance (0.5 * N(0,1), shuffled 2x pool, NaN
poisoning, atol = rtol = 2e-2):
- groups of 64 and 128 q-heads (the matrix-core scan in 4 and 8 chunks of 16);
- 16 to 64 kv-heads;
- cache blocks of 256 and 1024 tokens;
- sequences of 131072 tokens;
- batches of 8192 requests (the balanced launch's prefix table over several
  scan rounds) and of 65535 (the largest grid the launchers accept).
Every case runs v1 (single pass), v2 at a fixed split count and at the
automatic one, and the balanced launch where its group limit allows.
"""

import numpy as np
import pytest
import torch

import capi
from binding import KERNELS, gqa_decode_balanced, gqa_decode_v1, gqa_decode_v2
from cases import make_case
from gpu_util import assert_close, oracle
from test_gqa_decode import ATOL, RTOL, SCALE, ref_case

pytestmark = pytest.mark.gpu


def run_all(case, want, label, splits=(3,), balanced=True, v0=False):
    fns = [("v1", gqa_decode_v1)]
    fns += [(f"v2/ns{ns}", (lambda ns: lambda *a: gqa_decode_v2(*a, num_splits=ns))(ns))
            for ns in splits]
    fns.append(("v2/auto", lambda *a: gqa_decode_v2(*a, num_splits=0)))
    if balanced:
        fns.append(("balanced", gqa_decode_balanced))
    if v0:
        fns.append(("v0", KERNELS["v0"]))
    for name, fn in fns:
        print(f"{label} {name}", flush=True)
        out = fn(*case, SCALE)
        torch.cuda.synchronize()
        assert_close(out, want, ATOL, RTOL, f"{label}/{name}")


@pytest.mark.parametrize("Hq,Hkv", [(64, 1), (128, 1), (256, 2)])
def test_large_groups(gpu, Hq, Hkv):
    # Groups of 64 and 128: past the balanced launcher's limit of 16.
    case = ref_case(dict(S_list=[300, 1, 777], Hq=Hq, Hkv=Hkv, bs=16), seed=Hq + Hkv)
    run_all(case, oracle(case, SCALE), f"G{Hq // Hkv}", balanced=False, v0=True)


@pytest.mark.parametrize("Hq,Hkv", [(16, 16), (32, 32), (64, 64), (128, 32)])
def test_many_kv_heads(gpu, Hq, Hkv):
    case = ref_case(dict(S_list=[257, 40, 1000], Hq=Hq, Hkv=Hkv, bs=16), seed=Hq * Hkv)
    run_all(case, oracle(case, SCALE), f"Hkv{Hkv}")


@pytest.mark.parametrize("bs", [256, 1024])
def test_large_blocks(gpu, bs):
    case = ref_case(dict(S_list=[1, bs - 1, bs, 2 * bs + 5], Hq=32, Hkv=8, bs=bs), seed=bs)
    run_all(case, oracle(case, SCALE), f"bs{bs}", splits=(3, 16))


def test_long_sequences(gpu):
    # 131072 tokens: 16 splits of 8192 at the automatic count.
    case = ref_case(dict(S_list=[131072, 70000], Hq=8, Hkv=2, bs=64), seed=17)
    B, Hq, Hkv, bs, mb = 2, 8, 2, 64, case[3].shape[1]
    assert capi.pick_num_splits(B, Hq, Hkv, bs, mb, 0) >= 16
    run_all(case, oracle(case, SCALE), "S131072", splits=(64,))


def test_many_requests(gpu):
    # 8192 short ragged requests: the balanced launch's prefix table spans
    # several rounds of its scan; checked on every 37th request.
    S = np.random.default_rng(21).integers(1, 41, size=8192).tolist()
    case = ref_case(dict(S_list=S, Hq=8, Hkv=2, bs=16), seed=21)
    rows = list(range(0, 8192, 37)) + [8191]
    want = oracle(case, SCALE, rows)
    for name, fn in [("v1", gqa_decode_v1), ("v2/ns2", lambda *a: gqa_decode_v2(*a, num_splits=2)),
                     ("v2/auto", lambda *a: gqa_decode_v2(*a, num_splits=0)),
                     ("balanced", gqa_decode_balanced)]:
        print(f"B8192 {name}", flush=True)
        out = fn(*case, SCALE)
        torch.cuda.synchronize()
        assert_close(out[rows], want, ATOL, RTOL, f"B8192/{name}")


def test_largest_batch(gpu):
    # 65535 requests of 1-4 tokens: the largest batch the split launchers
    # accept (grid.y); 65536 is rejected before any launch.
    S = np.random.default_rng(23).integers(1, 5, size=65535).tolist()
    case = make_case(S, 4, 1, 4, pool_factor=1.5, seed=23, qkv_std=0.5)
    rows = list(range(0, 65535, 997)) + [65534]
    want = oracle(case, SCALE, rows)
    for name, fn in [("v1", gqa_decode_v1), ("v2/ns2", lambda *a: gqa_decode_v2(*a, num_splits=2))]:
        print(f"B65535 {name}", flush=True)
        out = fn(*case, SCALE)
        torch.cuda.synchronize()
        assert_close(out[rows], want, ATOL, RTOL, f"B65535/{name}")
    q, k, v, bt, sl = case
    big = torch.empty(65536, 4, 128, dtype=torch.bfloat16, device=q.device)
    rc = capi.v1_launch(big.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr(),
                        big.data_ptr(), 65536, 4, 1, 4, bt.shape[1], SCALE, None)
    assert rc == capi.HIP_ERROR_INVALID_VALUE
