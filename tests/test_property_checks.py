"""CPU checks of the properties tests/test_properties.py asserts on the GPU
at full size: each holds for the oracle (oracle/reference.py) on small
seeded ragged cases, and the exact ones catch the mistakes they are there
for, planted in copies of the oracle (swapped K and V, a dropped 1/l
normalisation, the scale applied twice). "Every token twice" is a
tolerance check of repeated block ids and doubled lengths; the oracle
comparisons of tests/test_configs.py cover wrong blocks.
"""

import numpy as np
import pytest

from oracle import reference as ref
from test_oracle import random_bf16_case

SCALE = 1.0 / np.sqrt(128.0)


def doubled(x):
    """bf16 bits of 2x (exact: a power-of-two scale of a finite bf16)."""
    return ref.f32_to_bf16(ref.bf16_to_f32(x) * np.float32(2))


def v_linear(attn, q, k, v, bt, sl):
    return np.array_equal(attn(q, k, doubled(v), bt, sl, SCALE), 2 * attn(q, k, v, bt, sl, SCALE))


def k_scale(attn, q, k, v, bt, sl):
    return np.array_equal(attn(q, doubled(k), v, bt, sl, SCALE / 2), attn(q, k, v, bt, sl, SCALE))


def convex(attn, q, k, v, bt, sl):
    out = attn(q, k, v, bt, sl, SCALE)
    G = q.shape[1] // k.shape[2]
    for b in range(q.shape[0]):
        _, V = ref.gather_kv(k, v, bt, int(sl[b]), b)
        lo = np.repeat(V.min(0), G, axis=0)
        hi = np.repeat(V.max(0), G, axis=0)
        slack = np.maximum(np.abs(lo), np.abs(hi)) * 2.0 ** -7 + 1e-6
        if (out[b] < lo - slack).any() or (out[b] > hi + slack).any():
            return False
    return True


def twice(attn, q, k, v, bt, sl):
    """Each request's blocks listed twice (then the -1 padding), twice the length."""
    bs = k.shape[1]
    assert all(s % bs == 0 for s in sl)
    bt2 = np.full((bt.shape[0], 2 * bt.shape[1]), -1, np.int32)
    for b, S in enumerate(sl):
        blocks = bt[b, :S // bs]
        bt2[b, :2 * len(blocks)] = np.concatenate([blocks, blocks])
    a = attn(q, k, v, bt, sl, SCALE)
    b = attn(q, k, v, bt2, sl * 2, SCALE)
    return np.allclose(a, b, atol=1e-5, rtol=1e-5)


PROPERTIES = {"v_linear": v_linear, "k_scale": k_scale, "convex": convex, "twice": twice}


# Planted mistakes, each a plausible slip in a decode kernel.
def swapped_kv(q, k, v, bt, sl, scale):
    return ref.attention_ref(q, v, k, bt, sl, scale)


def unnormalised(q, k, v, bt, sl, scale):
    out = np.zeros((q.shape[0], q.shape[1], 128), np.float32)
    G = q.shape[1] // k.shape[2]
    qf = ref.bf16_to_f32(q)
    for b in range(q.shape[0]):
        K, V = ref.gather_kv(k, v, bt, int(sl[b]), b)
        for h in range(q.shape[1]):
            s = (K[:, h // G] @ qf[b, h]) * np.float32(scale)
            out[b, h] = np.exp(s - s.max()) @ V[:, h // G]  # the 1/l is missing
    return out


def scale_twice(q, k, v, bt, sl, scale):
    return ref.attention_ref(q, k, v, bt, sl, scale * scale)


def case(seed, S_list, Hq=8, Hkv=2, bs=4):
    rng = np.random.default_rng(seed)
    return random_bf16_case(rng, S_list, Hq=Hq, Hkv=Hkv, bs=bs, poison=False)


@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("prop", list(PROPERTIES))
def test_oracle_has_property(seed, prop):
    assert PROPERTIES[prop](ref.attention_ref, *case(seed, [24, 8, 40]))


@pytest.mark.parametrize("mistake,prop", [(swapped_kv, "v_linear"), (swapped_kv, "k_scale"),
                                          (unnormalised, "convex"), (scale_twice, "k_scale")])
def test_property_catches_mistake(mistake, prop):
    assert not PROPERTIES[prop](mistake, *case(5, [24, 8, 40]))
