"""GPU tests of split launches whose grid leaves CUs idle.

With fewer (request, kv-head, split) workgroups than CUs, groups of up to 4
q-heads whose splits are at most 1024 tokens long run the matrix-core scan;
longer splits keep the VALU scan, with 8 or 12 waves per split where each
wave still gets two tiles; groups of 5 or more q-heads take the matrix-core
scan with 8 waves per split. The shapes below sit on both sides of the
1024-token boundary for each group size. Checked:
- every (request, q-head, split) workspace state against the oracle's state
  of the same token range, with NaN in every slot that must not be read;
- the output against the oracle;
- v2 with one split equal to v1 bit for bit;
- the single-launch form equal to partial + merge bit for bit.
"""

import pytest
import torch

from binding import gqa_decode_v1, gqa_decode_v2
from cases import make_case
from gpu_util import assert_close, oracle
from test_fused import counters, fused, fused_workspace, two_launch
from test_gqa_decode import SCALE
from test_split_range import check_states, partial

pytestmark = pytest.mark.gpu

# Split lengths per split count (32-token rounding): 1000 -> 1024 at one split
# (matrix-core side for small groups), 2100 -> 2112 / 1056 / 544 at 1 / 2 / 4
# splits (VALU, VALU, matrix-core), 17 -> one short split.
LENGTHS = [1000, 2100, 17]


@pytest.mark.parametrize("bs", [16, 7])
@pytest.mark.parametrize("G", [1, 4, 8])
@pytest.mark.parametrize("ns", [1, 2, 4])
def test_underfilled_states_and_output(gpu, G, ns, bs):
    Hkv = 8
    B = len(LENGTHS)
    assert B * Hkv * ns < torch.cuda.get_device_properties(0).multi_processor_count
    print(f"under-filled G={G} ns={ns} bs={bs}", flush=True)
    case = make_case(LENGTHS, G * Hkv, Hkv, bs, pool_factor=1.25, seed=G * 10 + ns, poison=True)
    ws, acc, m, l = partial(case, ns)
    check_states(case, acc, m, l, ns, list(range(B)))
    out = gqa_decode_v2(*case, SCALE, num_splits=ns)
    torch.cuda.synchronize()
    assert_close(out, oracle(case, SCALE), 2e-2, 2e-2, f"under-filled G={G} ns={ns} bs={bs}")
    if ns == 1:
        assert torch.equal(out, gqa_decode_v1(*case, SCALE)), "v2(ns=1) != v1 bitwise"


@pytest.mark.parametrize("G", [1, 4, 8])
@pytest.mark.parametrize("ns", [2, 4])
def test_underfilled_fused_equals_two_launches(gpu, G, ns):
    Hkv = 8
    B = len(LENGTHS)
    case = make_case(LENGTHS, G * Hkv, Hkv, 16, pool_factor=1.25, seed=G + ns, poison=True)
    ws, n = fused_workspace(B, G * Hkv, ns, case[0].device, fill=float("nan"))
    out = fused(case, ns, ws, n)
    want = two_launch(case, ns)
    torch.cuda.synchronize()
    assert torch.equal(out, want), f"G={G} ns={ns}: fused != partial + merge bitwise"
    assert not counters(ws, B, G * Hkv).any(), "arrival counters not left at zero"
