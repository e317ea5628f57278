"""GPU parity of the token-balanced split-KV launcher (gqa_decode_balanced_launch).

With 4 or 8 kv-heads the launcher runs the matrix-core scan (one wave per
kv-head; tests/test_balanced_mfma.py covers its groups of 5-16), with other
kv-head counts the VALU scan over (request, kv-head) segments: the tests
below run both, the reference's 8 kv-heads and the same groups over 16 (or 2
and 1) kv-heads.

Same inputs, poisoning and tolerance as the reference's kernel tests
(tests/test_gqa_decode.py:27-139 of the reference: 0.5 * N(0,1), shuffled 2x
pool, NaN in every slot that must not be read, atol = rtol = 2e-2), against
the oracle, through the C ABI with a caller-owned workspace. Covers the
reference's case grid for groups up to 4, block sizes that are not multiples
of 16, workgroup counts from 1 (no merge) to more workgroups than tiles
(empty shares), ragged batches with zero-length requests (NaN rows, the other
rows exact), batches longer than one prefix-scan round, bitwise
repeatability, and the G <= 4 BASELINE configs at full size (1e-2).
"""

import math

import numpy as np
import pytest
import torch

import capi
from binding import gqa_decode_balanced, gqa_decode_v1, gqa_decode_v2, prefer_balanced
from cases import config_seq_lens, make_case, make_config_case
from gpu_util import assert_close, numpy_oracle, oracle
from test_gqa_decode import CASES, ref_case

pytestmark = pytest.mark.gpu

ATOL = RTOL = 2e-2
SCALE = 1.0 / math.sqrt(128)


def balanced(case, scale=SCALE, nwg=0, out=None, parts=False):
    q, k, v, bt, sl = case
    B, Hq = q.shape[:2]
    Hkv, bs = k.shape[2], k.shape[1]
    nbytes = capi.balanced_workspace_bytes(B, Hq, Hkv, nwg)
    assert nbytes > 0
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device=q.device)
    out = torch.empty_like(q) if out is None else out
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr(), out.data_ptr(),
            B, Hq, Hkv, bs, bt.shape[1], scale, nwg, ws.data_ptr(), nbytes,
            torch.cuda.current_stream().cuda_stream)
    if parts:
        assert capi.balanced_partial_launch(*args) == 0
        assert capi.balanced_merge_launch(*args) == 0
    else:
        assert capi.balanced_launch(*args) == 0
    torch.cuda.synchronize()
    return out


GRID = {k: v for k, v in CASES.items() if v["Hq"] // v["Hkv"] <= 4}


@pytest.mark.parametrize("name", list(GRID))
@pytest.mark.parametrize("hkv", [8, 16])
def test_balanced_reference_grid(gpu, name, hkv):
    print(f"balanced {name} Hkv={hkv}", flush=True)
    cfg = dict(GRID[name])
    cfg["Hq"], cfg["Hkv"] = cfg["Hq"] // cfg["Hkv"] * hkv, hkv
    case = ref_case(cfg)
    assert_close(balanced(case), numpy_oracle(case, SCALE), ATOL, RTOL,
                 f"balanced/{name}/Hkv{hkv}")


@pytest.mark.parametrize("nwg", [1, 2, 3, 7, 64, 256, 1000])
def test_balanced_workgroup_counts(gpu, nwg):
    # 1: one share, every piece whole, no merge launch; 1000 > the 96 tiles of
    # the first case: most shares empty.
    print(f"balanced nwg={nwg}", flush=True)
    for cfg in (dict(S_list=[100, 257, 33, 1], Hq=32, Hkv=8, bs=16),
                dict(S_list=[4000, 17, 900], Hq=16, Hkv=4, bs=16),
                dict(S_list=[100, 257, 33, 1], Hq=64, Hkv=16, bs=16),
                dict(S_list=[4000, 17, 900], Hq=8, Hkv=2, bs=16)):
        case = ref_case(cfg, seed=nwg)
        assert_close(balanced(case, nwg=nwg), numpy_oracle(case, SCALE), ATOL, RTOL, f"nwg{nwg}")


@pytest.mark.parametrize("G", [1, 2, 3, 4])
@pytest.mark.parametrize("bs", [1, 7, 16, 24, 64])
@pytest.mark.parametrize("hkv", [4, 2, 1])
def test_balanced_groups_and_block_sizes(gpu, G, bs, hkv):
    print(f"balanced G={G} bs={bs} Hkv={hkv}", flush=True)
    cfg = dict(S_list=[1, 50, 333, 129, 700], Hq=hkv * G, Hkv=hkv, bs=bs)
    case = ref_case(cfg, seed=G * 100 + bs + hkv)
    assert_close(balanced(case, nwg=37), numpy_oracle(case, SCALE), ATOL, RTOL,
                 f"G{G}/bs{bs}/Hkv{hkv}")


@pytest.mark.parametrize("hkv", [8, 16])
def test_balanced_zero_length_requests(gpu, hkv):
    # seq_len 0 is unsupported (NaN, as in the reference); the other requests
    # must be unaffected, whichever share the empty ones fall into.
    S_list = [0, 37, 0, 0, 100, 0]
    case = make_case(S_list, 4 * hkv, hkv, 16, pool_factor=2, seed=5, qkv_std=0.5, poison=True)
    live = [i for i, s in enumerate(S_list) if s]
    for nwg in (1, 2, 5, 256):
        out = balanced(case, nwg=nwg).float().cpu()
        assert torch.isnan(out[[i for i, s in enumerate(S_list) if not s]]).all()
        assert_close(out[live].numpy(), oracle(case, SCALE, live), ATOL, RTOL, f"zero/nwg{nwg}")


@pytest.mark.parametrize("hkv", [8, 16])
def test_balanced_many_requests(gpu, hkv):
    # More requests than one prefix-scan round of the workgroup, short and
    # ragged.
    g = np.random.default_rng(3)
    S_list = [int(x) for x in g.integers(1, 300, size=700)]
    case = make_case(S_list, 4 * hkv, hkv, 16, pool_factor=1.2, seed=6, qkv_std=0.5,
                     poison=True)
    out = balanced(case)
    batches = list(range(0, 700, 7)) + [699]
    assert_close(out[batches], oracle(case, SCALE, batches), ATOL, RTOL, "many")


@pytest.mark.parametrize("hkv", [8, 16])
def test_balanced_repeatable(gpu, hkv):
    cfg = dict(S_list=[5000, 1, 2000, 777, 3333, 64], Hq=4 * hkv, Hkv=hkv, bs=16)
    case = ref_case(cfg, seed=9)
    first = balanced(case)
    for _ in range(3):
        assert torch.equal(balanced(case), first)


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c5"])
def test_balanced_configs(gpu, name):
    # BASELINE configs with 4-head groups at full size, north_star tolerance.
    print(f"balanced config {name}", flush=True)
    case = make_config_case(name, seed=0, poison=(name == "c5"))
    out = balanced(case)
    assert torch.isfinite(out.float()).all()
    B = case[0].shape[0]
    if name == "c5":
        S = config_seq_lens(name)
        order = np.argsort(S)
        batches = sorted({int(order[0]), int(order[-1]), 0, B - 1, B // 2, B // 3})
    else:
        batches = list(range(B))
    assert_close(out[batches], oracle(case, SCALE, batches), 1e-2, 1e-2, f"balanced/{name}")
    del case
    torch.cuda.empty_cache()


@pytest.mark.parametrize("hkv", [8, 16])
def test_balanced_parts_equal_launch(gpu, hkv):
    # Partial then merge, as two calls, is the combined launch.
    cfg = dict(S_list=[3000, 17, 900, 2500], Hq=4 * hkv, Hkv=hkv, bs=16)
    case = ref_case(cfg, seed=12)
    assert torch.equal(balanced(case, parts=True), balanced(case))


def test_balanced_ops(gpu):
    # The op, and v2's automatic choice where the rule prefers the balanced
    # launch, equal the C-ABI launch with one workgroup per CU bit for bit.
    S_list = [int(x) for x in np.random.default_rng(4).integers(1, 32768, size=24)]
    case = make_case(S_list, 32, 8, 16, pool_factor=1.1, seed=4, qkv_std=0.5)
    q, k, v, bt, sl = case
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert prefer_balanced(q.shape[0], 32, 8, 16, bt.shape[1], cus)
    want = balanced(case)
    assert torch.equal(gqa_decode_balanced(*case, SCALE), want)
    assert torch.equal(gqa_decode_v2(*case, SCALE, num_splits=0), want)
    assert torch.equal(gqa_decode_balanced(*case, SCALE, num_workgroups=7), balanced(case, nwg=7))
    with pytest.raises(RuntimeError, match="at most 16"):
        gqa_decode_balanced(torch.zeros(1, 136, 128, dtype=torch.bfloat16, device=q.device), k, v,
                            bt[:1], sl[:1], SCALE)


@pytest.mark.parametrize("seed", range(10))
def test_random_shapes(gpu, seed):
    # Seeded random combinations the fixed grids do not pair up: 1-6
    # requests of 1-3000 tokens, 1-16 kv-heads of 1-16 q-heads each, block
    # sizes 1-128 (multiples of 16 and not), NaN in every slot no request
    # owns; through v1, v2 at its automatic choice and at 1-40 splits, and the
    # balanced launch with 1-400 workgroups where it serves the shape (groups
    # of up to 4, or up to 16 with 4 or 8 kv-heads; elsewhere its workspace
    # size is 0), all against the oracle.
    rng = np.random.default_rng(2000 + seed)
    B = int(rng.integers(1, 7))
    Hkv = int(rng.choice([1, 2, 4, 8, 16]))
    G = int(rng.integers(1, 17))
    bs = int(rng.choice([1, 7, 16, 24, 32, 64, 128]))
    S_list = [int(x) for x in rng.integers(1, 3001, size=B)]
    ns = int(rng.integers(1, 41))
    nwg = int(rng.integers(1, 401))
    print(f"random seed={seed}: B={B} Hq={G * Hkv} Hkv={Hkv} bs={bs} ns={ns} nwg={nwg} "
          f"S={S_list}", flush=True)
    case = ref_case(dict(S_list=S_list, Hq=G * Hkv, Hkv=Hkv, bs=bs), seed=seed)
    want = numpy_oracle(case, SCALE)
    label = f"random{seed}"
    assert_close(gqa_decode_v1(*case, SCALE), want, ATOL, RTOL, f"{label}/v1")
    assert_close(gqa_decode_v2(*case, SCALE, num_splits=0), want, ATOL, RTOL, f"{label}/auto")
    assert_close(gqa_decode_v2(*case, SCALE, num_splits=ns), want, ATOL, RTOL, f"{label}/ns{ns}")
    if G <= 4 or Hkv in (4, 8):
        assert_close(balanced(case, nwg=nwg), want, ATOL, RTOL, f"{label}/bal{nwg}")
    else:
        assert capi.balanced_workspace_bytes(B, G * Hkv, Hkv, nwg) == 0


@pytest.mark.parametrize("kind", ["v2_ns1", "v2_ns8", "balanced", "balanced_noalloc"])
def test_graph_replay(gpu, kind):
    # The C-ABI launches captured once in a HIP graph and replayed, as a
    # serving loop runs them: each replay (on new queries written between
    # replays, with the eager launch itself in between) equals the eager
    # launch on the same inputs bit for bit. None of these launches records a
    # memset or allocates.
    case = ref_case(dict(S_list=[700, 64, 3000, 1, 2000], Hq=32, Hkv=8, bs=16), seed=21)
    q, k, v, bt, sl = case
    B, Hq = q.shape[:2]
    Hkv, bs, mb = k.shape[2], k.shape[1], bt.shape[1]
    ptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr())

    def make_launch(out):
        if kind.startswith("v2"):
            ns = int(kind[len("v2_ns"):])
            acc = torch.empty(B * Hq * ns * 128, dtype=torch.float32, device=q.device)
            m = torch.empty(B * Hq * ns, dtype=torch.float32, device=q.device)
            l = torch.empty(B * Hq * ns, dtype=torch.float32, device=q.device)
            return lambda: capi.v2_launch(*ptrs, out.data_ptr(), B, Hq, Hkv, bs, mb, SCALE, ns,
                                          acc.data_ptr(), m.data_ptr(), l.data_ptr(),
                                          torch.cuda.current_stream().cuda_stream)
        if kind == "balanced":
            nbytes = capi.balanced_workspace_bytes(B, Hq, Hkv, 0)
            ws = torch.empty(nbytes // 4, dtype=torch.float32, device=q.device)
            return lambda: capi.balanced_launch(*ptrs, out.data_ptr(), B, Hq, Hkv, bs, mb, SCALE, 0,
                                                ws.data_ptr(), nbytes,
                                                torch.cuda.current_stream().cuda_stream)
        return lambda: capi.balanced_launch_noalloc(*ptrs, out.data_ptr(), B, Hq, Hkv, bs, mb,
                                                    SCALE, 0,
                                                    torch.cuda.current_stream().cuda_stream)

    out = torch.empty_like(q)
    launch = make_launch(out)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        assert launch() == 0  # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        assert launch() == 0
    eager_out = torch.empty_like(q)
    eager = make_launch(eager_out)
    gen = torch.Generator(device="cpu").manual_seed(22)
    for rep in range(4):
        q.copy_((0.5 * torch.randn(q.shape, generator=gen)).to(q.device, torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        assert eager() == 0
        torch.cuda.synchronize()
        assert torch.equal(out, eager_out), f"{kind}: replay {rep} differs from the eager launch"
    assert_close(out, numpy_oracle(case, SCALE), ATOL, RTOL, f"{kind}/graph")
