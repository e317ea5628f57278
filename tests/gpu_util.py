"""Helpers shared by the GPU parity tests: host copies of device cases and the
oracle calls on them (the oracle is the checker; the kernels are what run)."""

import numpy as np
import torch

from cases import bits, host_case  # noqa: F401  (re-exported for the tests)
from oracle import c_oracle
from oracle import reference as ref

D = 128


def oracle(case, scale, batches=None):
    """fp32 reference output [len(batches) or B, Hq, 128] from the C oracle."""
    return c_oracle.attention_ref(*host_case(case, batches), scale)


def numpy_oracle(case, scale):
    return ref.attention_ref(*host_case(case), scale)


def assert_close(out, want, atol, rtol, label=""):
    got = out.float().cpu().numpy() if isinstance(out, torch.Tensor) else out
    assert np.isfinite(want).all(), "oracle output not finite"
    bad = ~np.isclose(got, want, atol=atol, rtol=rtol)
    if bad.any():
        err = np.abs(got - want)
        rel = err / np.maximum(np.abs(want), 1e-8)
        idx = np.unravel_index(np.argmax(np.where(bad, err, 0)), got.shape)
        raise AssertionError(
            f"{label} mismatch: {bad.sum()} of {bad.size} outside atol={atol} rtol={rtol}; "
            f"max-abs={err.max():.3e} max-rel={rel.max():.3e}; worst at {idx}: "
            f"got {got[idx]!r} want {want[idx]!r}")
