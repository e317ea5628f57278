"""CPU checks of the balanced MLA launch plan as the Python surface reports it
(mla.get_mla_metadata's num_splits), against a direct simulation of the
share walk the split kernel performs: share w of n takes tiles
[w T / n, (w + 1) T / n) of the request-ordered 32-token tiles, n = min(CUs
per row group, T), and every request gets one partial result per share that
holds some of its tiles."""

import pytest
import torch

from mla import get_mla_metadata


def simulate(S_list, n_share):
    tiles = [max(s, 0) // 32 + (1 if max(s, 0) % 32 else 0) for s in S_list]
    T = sum(tiles)
    n = min(n_share, T)
    pieces = [0] * len(S_list)
    pre = [0]
    for t in tiles:
        pre.append(pre[-1] + t)
    for w in range(n):
        t0, t1 = w * T // n, (w + 1) * T // n
        for b in range(len(S_list)):
            if max(pre[b], t0) < min(pre[b + 1], t1):
                pieces[b] += 1
    out = [0]
    for p in pieces:
        out.append(out[-1] + p)
    return out


@pytest.mark.parametrize("S_list,rows", [([4096] * 8, 128), ([0, 1, 33, 0, 5000], 128),
                                         ([100000], 128), ([31, 32, 33] * 50, 256),
                                         ([0, 0], 64), ([7000, 1, 1, 1, 9000], 300)])
def test_plan_pieces(S_list, rows):
    sl = torch.tensor(S_list, dtype=torch.int32)
    meta, splits = get_mla_metadata(sl, rows, 1)
    assert int(meta[0, 0]) == 0
    nwg = int(meta[0, 1])
    groups = -(-rows // 128)
    assert splits.tolist() == simulate(S_list, max(1, nwg // groups))


def test_fixed_plan():
    sl = torch.tensor([100, 2000, 0], dtype=torch.int32)
    meta, splits = get_mla_metadata(sl, 128, 1, num_splits=4)
    assert int(meta[0, 0]) == 4 and splits.tolist() == [0, 4, 8, 12]
    with pytest.raises(ValueError):
        get_mla_metadata(sl, 128, 2)


@pytest.mark.parametrize("B,s_q,h_q,cus,want", [(32, 1, 128, 256, 8), (64, 1, 128, 256, 4),
                                                (128, 1, 128, 256, 2), (1, 1, 128, 256, 128),
                                                (8, 2, 128, 256, 16), (3, 1, 200, 256, 43),
                                                (256, 1, 64, 256, 1), (300, 1, 128, 256, 1)])
def test_pick_num_splits_covers_cus(B, s_q, h_q, cus, want):
    # The (row group, request, split) grid covers num_cus workgroups with the
    # fewest splits: B * ceil(s_q h_q / 128) row groups per split. Long
    # sequences (1 << 20 tokens), so the 256-token minimum does not bind.
    import capi

    ns = capi.mla_pick_num_splits(B, s_q, h_q, 64, (1 << 20) // 64, cus)
    groups = B * -(-(s_q * h_q) // 128)
    assert ns == want
    assert ns == 128 or groups * ns >= cus  # 128: MLA_DECODE_MAX_SPLITS
    assert ns == 1 or groups * (ns - 1) < cus


def test_pick_num_splits_min_chunk():
    import capi

    # 1000 tokens (125 blocks of 8): at most 1000 // 256 = 3 splits, however
    # few the requests; 128 tokens: one.
    assert capi.mla_pick_num_splits(1, 1, 128, 8, 125, 256) == 3
    assert capi.mla_pick_num_splits(1, 1, 128, 64, 2, 256) == 1
