"""GPU parity tests of the matrix-core scan's slot-group layout.

Groups of 5-16 q-heads over 4 or 8 kv-heads run the matrix-core scan with one
workgroup per (split, request) and one wave per kv-head whenever the grid
gives at least 3/4 of the CUs eight resident waves. The small cases of the
reference's grid (tests/test_gqa_decode.py) never fill the chip, so these
tests pick batch and split counts from the device's CU count that do, and
check the layout the way the reference checks its kernels: outputs against
the fp32 oracle on ragged, NaN-poisoned inputs (atol = rtol = 2e-2), every
split's workspace state against the oracle's state of the same token range,
the single pass (v1, and v2 with one split, bitwise equal), block sizes off
the 16-token tile, and run-to-run bitwise determinism.
"""

import numpy as np
import pytest
import torch

import capi
from binding import gqa_decode_v1, gqa_decode_v2
from gpu_util import host_case, oracle
from oracle import reference as ref
from test_gqa_decode import (SCALE, W_REL, alloc_ws, build_segments, ref_case, run_and_check,
                             stream_ptr)

pytestmark = pytest.mark.gpu


def cu_count():
    return torch.cuda.get_device_properties(0).multi_processor_count


def slot_splits(B, Hkv):
    """Fewest splits whose grid takes the slot-group layout: B * ns * Hkv
    waves of which at least 3/4 of 8 per CU."""
    return -(-(24 * cu_count()) // (4 * B * Hkv))


def slot_batch(Hkv):
    """Fewest requests that take the layout with a single split."""
    return -(-(24 * cu_count()) // (4 * Hkv))


def ragged(B, seed, s_max=700):
    """Seeded lengths in [1, s_max] with one token, exact blocks and a
    partial block among them."""
    S = np.random.default_rng(seed).integers(1, s_max + 1, size=B).tolist()
    S[:3] = [1, 64, 65]
    return S


SHAPES = [(64, 8, 16), (40, 8, 16), (48, 8, 64), (128, 8, 16), (64, 8, 7), (32, 4, 16),
          (64, 4, 64), (20, 4, 7)]


@pytest.mark.parametrize("Hq,Hkv,bs", SHAPES)
def test_slot_layout_matches_oracle(gpu, Hq, Hkv, bs):
    B = 24 if Hkv == 8 else 48
    ns = slot_splits(B, Hkv)
    print(f"slot layout Hq={Hq} Hkv={Hkv} bs={bs} B={B} ns={ns}", flush=True)
    case = ref_case(dict(S_list=ragged(B, seed=Hq + bs), Hq=Hq, Hkv=Hkv, bs=bs), seed=Hq)
    run_and_check(lambda *a: gqa_decode_v2(*a, num_splits=ns), case, want=oracle(case, SCALE),
                  label=f"slot Hq{Hq}/Hkv{Hkv}/bs{bs}")


def test_slot_partial_states_match_oracle(gpu):
    """Each (b, q-head, split) workspace state of the slot-group launch
    against the oracle's state of the same token range."""
    Hq, Hkv, bs, B = 64, 8, 16, 12
    ns = slot_splits(B, Hkv)
    case = ref_case(dict(S_list=ragged(B, seed=5, s_max=400), Hq=Hq, Hkv=Hkv, bs=bs), seed=5)
    q, k, v, bt, sl = case
    ws, acc, m, l = alloc_ws(B, Hq, ns, q.device)
    ws.fill_(float("nan"))
    rc = capi.v2_partial_launch(q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(),
                                sl.data_ptr(), B, Hq, Hkv, bs, bt.shape[1], SCALE, ns,
                                acc.data_ptr(), m.data_ptr(), l.data_ptr(), stream_ptr())
    assert rc == 0
    torch.cuda.synchronize()
    G = Hq // Hkv
    qh, kh, vh, bth, slh = host_case(case)
    acc_h, m_h, l_h = acc.cpu().numpy(), m.cpu().numpy(), l.cpu().numpy()
    for b in range(B):
        K, V = ref.gather_kv(kh, vh, bth, int(slh[b]), b)
        for h in range(Hq):
            for i, (a, e) in enumerate(build_segments(int(slh[b]), ns)):
                if a == e:
                    assert m_h[b, h, i] == -np.inf and l_h[b, h, i] == 0
                    assert not acc_h[b, h, i].any()
                    continue
                mw, lw, aw = ref.partial_state(ref.bf16_to_f32(qh[b, h]), K[a:e, h // G],
                                               V[a:e, h // G], SCALE)
                assert m_h[b, h, i] == pytest.approx(mw, abs=1e-5)
                assert l_h[b, h, i] == pytest.approx(lw, rel=W_REL)
                vmax = float(np.abs(V[a:e, h // G]).max())
                np.testing.assert_allclose(acc_h[b, h, i], aw, rtol=0, atol=W_REL * lw * vmax)


@pytest.mark.parametrize("Hkv", [8, 4])
def test_slot_single_pass(gpu, Hkv):
    """Enough requests take the layout with one split: v1 and v2(num_splits=1)
    run the same single pass and agree bit for bit."""
    Hq, bs = 8 * Hkv, 16
    B = slot_batch(Hkv)
    S = np.random.default_rng(Hkv).integers(1, 80, size=B).tolist()
    case = ref_case(dict(S_list=S, Hq=Hq, Hkv=Hkv, bs=bs), seed=Hkv)
    want = oracle(case, SCALE)
    out1 = run_and_check(gqa_decode_v1, case, want=want, label="slot v1")
    out2 = run_and_check(lambda *a: gqa_decode_v2(*a, num_splits=1), case, want=want,
                         label="slot v2 ns=1")
    assert torch.equal(out1, out2), "v2(num_splits=1) != v1 bitwise"


def test_slot_bitwise_deterministic(gpu):
    Hq, Hkv, bs, B = 64, 8, 16, 24
    ns = slot_splits(B, Hkv)
    case = ref_case(dict(S_list=ragged(B, seed=9), Hq=Hq, Hkv=Hkv, bs=bs), seed=9)
    first = gqa_decode_v2(*case, SCALE, num_splits=ns)
    for _ in range(4):
        assert torch.equal(gqa_decode_v2(*case, SCALE, num_splits=ns), first)


def test_heuristic_takes_slot_layout(gpu):
    """The automatic split count for BASELINE config 4's shape (64Q/8KV,
    B=32, S=32768, block 64) gives the slot-group grid."""
    cus = cu_count()
    ns = capi.pick_num_splits(32, 64, 8, 64, 512, cus)
    assert 32 * ns * 8 * 4 >= 24 * cus
