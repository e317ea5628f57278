"""The page-table adapter and the vendor-library baseline.

block_table_to_paged is checked against the reference's known-answer vector
(tests/test_flashinfer_baseline.py:20-31, transcribed into
tests/golden/notes_w1_kat.json) and by brute force on random ragged tables;
the SDPA baseline is checked against the oracle on the reference's baseline
cases (tests/test_flashinfer_baseline.py:34-52) with its tolerance (2e-2):
on the CPU (torch's CPU flash backend) and, marked gpu, on the MI355X
(AOTriton).
"""

import json
import math
import os

import numpy as np
import pytest
import torch

from baselines.paged import block_table_to_paged, pages_per_request, paged_to_block_table
from baselines.sdpa_adapter import make_sdpa_runner, sdpa_decode
from cases import host_case, make_case
from oracle import reference as ref

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "notes_w1_kat.json")
SCALE = 1.0 / math.sqrt(128)
ATOL = RTOL = 2e-2

# The reference's baseline cases (tests/test_flashinfer_baseline.py:34-36,
# shapes from tests/test_gqa_decode.py:89-98) plus one uniform batch, which
# takes the single-call path the matrix times.
BASELINE_CASES = {
    "a_base": dict(S_list=[100, 257, 512, 33], Hq=32, Hkv=8, bs=16),
    "e_partial_blocks": dict(S_list=[17, 65], Hq=32, Hkv=8, bs=16),
    "g_hq64": dict(S_list=[100, 257, 512, 33], Hq=64, Hkv=8, bs=16),
    "f_bs64": dict(S_list=[100, 257, 512, 33], Hq=32, Hkv=8, bs=64),
    "uniform": dict(S_list=[300, 300, 300], Hq=32, Hkv=8, bs=16),
}


def kat():
    with open(GOLDEN) as f:
        return json.load(f)["block_table_to_paged"]


def check_kat(device):
    k = kat()
    bt = torch.tensor(k["block_table"], dtype=torch.int32, device=device)
    sl = torch.tensor(k["seq_lens"], dtype=torch.int32, device=device)
    indptr, indices, last = block_table_to_paged(bt, sl, k["page_size"])
    assert indptr.tolist() == k["indptr"]
    assert indices.tolist() == k["indices"]
    assert last.tolist() == k["last_page_len"]
    for t in (indptr, indices, last):
        assert t.dtype == torch.int32 and t.device == bt.device


def test_block_table_to_paged_kat():
    check_kat("cpu")


@pytest.mark.parametrize("seed", range(5))
@pytest.mark.parametrize("bs", [1, 16, 64])
def test_block_table_to_paged_brute_force(seed, bs):
    g = np.random.default_rng(seed)
    B = int(g.integers(1, 9))
    S = g.integers(1, 40 * bs + 1, size=B)
    n = [(int(s) + bs - 1) // bs for s in S]
    width = max(n) + int(g.integers(0, 3))
    ids = g.permutation(sum(n) + 5)
    table = np.full((B, width), -1, dtype=np.int32)
    off = 0
    for b in range(B):
        table[b, :n[b]] = ids[off:off + n[b]]
        off += n[b]
    indptr, indices, last = block_table_to_paged(torch.from_numpy(table),
                                                 torch.from_numpy(S.astype(np.int32)), bs)
    want_ptr = np.concatenate([[0], np.cumsum(n)])
    assert indptr.tolist() == want_ptr.tolist()
    assert indices.tolist() == [int(table[b, j]) for b in range(B) for j in range(n[b])]
    assert last.tolist() == [int(S[b]) - (n[b] - 1) * bs for b in range(B)]
    assert all(1 <= x <= bs for x in last.tolist())
    back = paged_to_block_table(indptr, indices, width)
    assert torch.equal(back, torch.from_numpy(table))


def test_pages_per_request():
    sl = torch.tensor([1, 15, 16, 17, 32, 33], dtype=torch.int32)
    assert pages_per_request(sl, 16).tolist() == [1, 1, 1, 2, 2, 3]
    with pytest.raises(ValueError):
        pages_per_request(sl, 0)


def test_block_table_to_paged_rejects_bad_input():
    bt = torch.zeros(2, 2, dtype=torch.int32)
    with pytest.raises(ValueError):
        block_table_to_paged(bt, torch.tensor([16, 33], dtype=torch.int32), 16)  # 3 pages > 2
    with pytest.raises(ValueError):
        block_table_to_paged(bt, torch.tensor([1], dtype=torch.int32), 16)
    with pytest.raises(ValueError):
        paged_to_block_table(torch.tensor([0, 3]), torch.arange(3), max_blocks=2)


def baseline_case(name, device, seed=0):
    c = BASELINE_CASES[name]
    nb = sum((s + c["bs"] - 1) // c["bs"] for s in c["S_list"])
    return make_case(c["S_list"], c["Hq"], c["Hkv"], c["bs"], pool=2 * nb, seed=seed,
                     qkv_std=0.5, poison=True, device=device)


def check_baseline(case, backend):
    out = sdpa_decode(*case, SCALE, backend=backend)
    if out.is_cuda:
        torch.cuda.synchronize()
    want = ref.attention_ref(*host_case(case), SCALE)
    got = out.float().cpu().numpy()
    assert out.dtype == torch.bfloat16 and out.shape == case[0].shape
    assert np.isfinite(got).all()
    err = np.abs(got - want)
    assert np.allclose(got, want, atol=ATOL, rtol=RTOL), f"max-abs {err.max():.3e}"


@pytest.mark.parametrize("name", list(BASELINE_CASES))
def test_sdpa_baseline_cpu(name):
    check_baseline(baseline_case(name, "cpu"), "flash")


def test_sdpa_baseline_empty_batch():
    q, k, v, bt, sl = baseline_case("uniform", "cpu")
    out = make_sdpa_runner(q[:0], k, v, bt[:0], sl[:0], SCALE)()
    assert out.shape == (0, 32, 128)


@pytest.mark.gpu
def test_block_table_to_paged_gpu(gpu):
    check_kat(gpu)


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(BASELINE_CASES))
def test_sdpa_baseline_gpu(gpu, name):
    print(f"sdpa baseline {name}", flush=True)
    check_baseline(baseline_case(name, gpu), "auto")


@pytest.mark.parametrize("name", ["a_base", "g_hq64", "f_bs64"])
def test_bench_spot_check_reference(name):
    # The benchmark tools' fp32 torch reference (used for their spot checks)
    # against the oracle; it must agree to fp32 rounding.
    import cases

    case = baseline_case(name, "cpu")
    got = cases.torch_ref_fp32(*case, SCALE, range(case[0].shape[0])).numpy()
    want = ref.attention_ref(*host_case(case), SCALE)
    np.testing.assert_allclose(got, want, atol=1e-5, rtol=1e-5)
