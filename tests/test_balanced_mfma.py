"""GPU parity of the token-balanced launch for groups of 5-16 q-heads.

For these groups gqa_decode_balanced_launch runs the matrix-core scan with
one wave per kv-head (4 or 8 kv-heads) and splits the batch's requests, not
its (request, kv-head) segments, into equal token shares. Same inputs,
poisoning and tolerance as the reference's kernel tests (0.5 * N(0,1),
shuffled 2x pool, NaN in every slot that must not be read, atol = rtol =
2e-2), against the oracle, through the C ABI with a caller-owned workspace:
group sizes 5-16 over 8 and 4 kv-heads, block sizes off the 16-token tile,
workgroup counts from 1 (no merge) to more workgroups than tiles (empty
shares), zero-length requests, the two halves against the whole launch,
bitwise repeatability, the op against the C ABI, and BASELINE config 4 plus
a ragged 64Q/8KV batch at full size (1e-2).
"""

import math

import numpy as np
import pytest
import torch

from binding import gqa_decode_balanced
from cases import make_case, make_config_case
from gpu_util import assert_close, numpy_oracle, oracle
from test_balanced import balanced
from test_gqa_decode import CASES, ref_case

pytestmark = pytest.mark.gpu

ATOL = RTOL = 2e-2
SCALE = 1.0 / math.sqrt(128)


def test_balanced_mfma_reference_case(gpu):
    case = ref_case(CASES["g_hq64"])
    assert_close(balanced(case), numpy_oracle(case, SCALE), ATOL, RTOL, "balanced/g_hq64")


@pytest.mark.parametrize("G,Hkv", [(5, 8), (8, 8), (16, 8), (6, 4), (8, 4), (16, 4)])
@pytest.mark.parametrize("bs", [7, 16, 64])
def test_balanced_mfma_groups_and_block_sizes(gpu, G, Hkv, bs):
    print(f"balanced mfma G={G} Hkv={Hkv} bs={bs}", flush=True)
    cfg = dict(S_list=[1, 50, 333, 129, 700, 16, 65], Hq=G * Hkv, Hkv=Hkv, bs=bs)
    case = ref_case(cfg, seed=G * 100 + bs + Hkv)
    assert_close(balanced(case, nwg=37), oracle(case, SCALE), ATOL, RTOL,
                 f"mfma G{G}/Hkv{Hkv}/bs{bs}")


@pytest.mark.parametrize("nwg", [1, 2, 3, 7, 64, 256, 1000])
def test_balanced_mfma_workgroup_counts(gpu, nwg):
    # 1: one share, every piece whole, no merge launch; 1000 > the 199 tiles:
    # most shares empty.
    print(f"balanced mfma nwg={nwg}", flush=True)
    case = ref_case(dict(S_list=[1000, 257, 33, 1, 1900], Hq=64, Hkv=8, bs=16), seed=nwg)
    assert_close(balanced(case, nwg=nwg), oracle(case, SCALE), ATOL, RTOL, f"mfma nwg{nwg}")


def test_balanced_mfma_zero_length_requests(gpu):
    S_list = [0, 37, 0, 0, 100, 0, 2000]
    case = make_case(S_list, 64, 8, 16, pool_factor=2, seed=5, qkv_std=0.5, poison=True)
    live = [i for i, s in enumerate(S_list) if s]
    for nwg in (1, 2, 5, 256):
        out = balanced(case, nwg=nwg).float().cpu()
        assert torch.isnan(out[[i for i, s in enumerate(S_list) if not s]]).all()
        assert_close(out[live].numpy(), oracle(case, SCALE, live), ATOL, RTOL,
                     f"mfma zero/nwg{nwg}")


def test_balanced_mfma_parts_and_repeatable(gpu):
    case = ref_case(dict(S_list=[5000, 1, 2000, 777, 3333, 64], Hq=64, Hkv=8, bs=16), seed=9)
    first = balanced(case)
    assert torch.equal(balanced(case, parts=True), first)
    for _ in range(3):
        assert torch.equal(balanced(case), first)


def test_balanced_mfma_op(gpu):
    case = ref_case(dict(S_list=[3000, 17, 900, 2500], Hq=64, Hkv=8, bs=16), seed=12)
    assert torch.equal(gqa_decode_balanced(*case, SCALE), balanced(case))
    assert torch.equal(gqa_decode_balanced(*case, SCALE, num_workgroups=7), balanced(case, nwg=7))


def test_balanced_mfma_config4(gpu):
    # BASELINE config 4 (64Q/8KV, B=32, S=32768, block 64) at full size.
    print("balanced mfma config c4", flush=True)
    case = make_config_case("c4", seed=0)
    out = balanced(case)
    batches = [0, 7, 31]
    assert_close(out[batches], oracle(case, SCALE, batches), 1e-2, 1e-2, "balanced/c4")
    del case
    torch.cuda.empty_cache()


def test_balanced_mfma_ragged(gpu):
    # A ragged 64Q/8KV batch, lengths up to 32768, garbage (NaN) in every slot
    # that must not be read.
    print("balanced mfma ragged", flush=True)
    S_list = [int(x) for x in np.random.default_rng(7).integers(1, 32769, size=32)]
    case = make_case(S_list, 64, 8, 64, pool_factor=1.25, seed=7, poison=True)
    out = balanced(case)
    order = np.argsort(S_list)
    batches = sorted({int(order[0]), int(order[-1]), 0, 31, 15})
    assert_close(out[batches], oracle(case, SCALE, batches), 1e-2, 1e-2, "balanced/ragged64")
    del case
    torch.cuda.empty_cache()
