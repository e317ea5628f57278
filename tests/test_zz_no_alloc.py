"""GPU tests of the allocation-free token-balanced launch
(gqa_decode_balanced_launch_noalloc), through the C ABI.

Its kernels are gqa_decode_balanced_launch's, run on the library's own
per-device scratch array instead of a caller workspace, so with the same
num_workgroups the two give the same bits. Checked on two calls in a row, the
second with a smaller batch (it runs on what the first left in the shared
array), for the matrix-core scan (4 and 8 kv-heads) and the VALU scan (other
kv-head counts); the smaller batch also against the fp32 oracle. Host-side
rejections launch nothing: a workspace beyond the array's 32 MiB gives
hipErrorOutOfMemory, an empty batch succeeds.
"""

import math

import numpy as np
import pytest
import torch

import capi
from cases import make_case
from gpu_util import assert_close, oracle

pytestmark = pytest.mark.gpu

SCALE = 1.0 / math.sqrt(128)
HIP_ERROR_OUT_OF_MEMORY = 2


def shape(case):
    q, k, _, bt, _ = case
    return q.shape[0], q.shape[1], k.shape[2], k.shape[1], bt.shape[1]


def ptrs(case):
    return tuple(t.data_ptr() for t in case)


def with_workspace(case, nwg):
    B, Hq, Hkv, bs, mb = shape(case)
    out = torch.empty_like(case[0])
    n = capi.balanced_workspace_bytes(B, Hq, Hkv, nwg)
    ws = torch.empty(n, dtype=torch.uint8, device=case[0].device)
    rc = capi.balanced_launch(*ptrs(case), out.data_ptr(), B, Hq, Hkv, bs, mb, SCALE, nwg,
                              ws.data_ptr(), n, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    return out


def no_alloc(case, nwg):
    B, Hq, Hkv, bs, mb = shape(case)
    out = torch.empty_like(case[0])
    rc = capi.balanced_launch_noalloc(*ptrs(case), out.data_ptr(), B, Hq, Hkv, bs, mb, SCALE, nwg,
                                      torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    return out


@pytest.mark.parametrize("Hq,Hkv,nwg", [(32, 8, 0), (64, 8, 256), (16, 4, 100), (32, 16, 0),
                                        (8, 2, 37)])
def test_noalloc_equals_workspace_launch(gpu, Hq, Hkv, nwg):
    rng = np.random.default_rng(Hq + Hkv)
    big = rng.integers(1, 6000, size=24).tolist()
    small = rng.integers(1, 900, size=5).tolist()
    for step, S in enumerate((big, small)):
        print(f"no-alloc Hq={Hq} Hkv={Hkv} nwg={nwg} call {step}: B={len(S)}", flush=True)
        case = make_case(S, Hq, Hkv, 16, pool_factor=1.25, seed=step, qkv_std=0.5, poison=True)
        got = no_alloc(case, nwg)
        want = with_workspace(case, nwg)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {step}: differs from the workspace launch"
        if step == 1:
            assert_close(got, oracle(case, SCALE), 1e-2, 1e-2, f"no-alloc Hq{Hq}/Hkv{Hkv}")


def test_noalloc_rejects_oversize_and_accepts_empty(gpu):
    case = make_case([300, 17], 128, 8, 16, pool_factor=1.25, seed=3, qkv_std=0.5)
    B, Hq, Hkv, bs, mb = shape(case)
    out = torch.full_like(case[0], 7.0)
    sp = torch.cuda.current_stream().cuda_stream
    # 256 workgroups x 2 states x 128 q-heads: 34.6 MB of workspace, over 32 MiB.
    assert capi.balanced_workspace_bytes(B, Hq, Hkv, 256) > capi.NOALLOC_SCRATCH_BYTES
    rc = capi.balanced_launch_noalloc(*ptrs(case), out.data_ptr(), B, Hq, Hkv, bs, mb, SCALE, 256,
                                      sp)
    assert rc == HIP_ERROR_OUT_OF_MEMORY
    torch.cuda.synchronize()
    assert (out.float() == 7.0).all(), "a rejected call must launch nothing"
    # The same batch at 64 workgroups fits and matches the workspace launch.
    assert torch.equal(no_alloc(case, 64), with_workspace(case, 64))
    assert capi.balanced_launch_noalloc(*ptrs(case), out.data_ptr(), 0, Hq, Hkv, bs, mb, SCALE, 0,
                                        sp) == 0


# Run in a fresh process, so that no call has resolved the device's scratch
# array yet: the first call, made while the stream is captured into a graph,
# is refused with hipErrorStreamCaptureUnsupported and launches nothing; after
# one eager call, calls captured into a graph replay to the eager result.
FIRST_CALL_UNDER_CAPTURE = r"""
import math, sys
import torch
sys.path[:0] = {paths!r}
import capi
from cases import make_case
case = make_case([700, 33, 2000], 32, 8, 16, pool_factor=1.25, seed=5, qkv_std=0.5)
q, k, v, bt, sl = case
B, Hq, Hkv, bs, mb = q.shape[0], q.shape[1], k.shape[2], k.shape[1], bt.shape[1]
scale = 1.0 / math.sqrt(128)
args = tuple(t.data_ptr() for t in case)
out = torch.full_like(q, 3.0)
s = torch.cuda.Stream()
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=s):
    rc_first = capi.balanced_launch_noalloc(*args, out.data_ptr(), B, Hq, Hkv, bs, mb, scale, 64,
                                            s.cuda_stream)
torch.cuda.synchronize()
assert rc_first == 900, rc_first
assert (out.float() == 3.0).all(), "a refused call must launch nothing"
eager = torch.empty_like(q)
assert capi.balanced_launch_noalloc(*args, eager.data_ptr(), B, Hq, Hkv, bs, mb, scale, 64,
                                    0) == 0
torch.cuda.synchronize()
g2 = torch.cuda.CUDAGraph()
with torch.cuda.graph(g2, stream=s):
    rc = capi.balanced_launch_noalloc(*args, out.data_ptr(), B, Hq, Hkv, bs, mb, scale, 64,
                                      s.cuda_stream)
assert rc == 0, rc
for _ in range(3):
    out.fill_(0.0)
    g2.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, eager), "replay differs from the eager call"
print("FIRST_CALL_UNDER_CAPTURE_OK", flush=True)
"""


def test_noalloc_first_call_under_capture(gpu):
    import os
    import subprocess
    import sys

    here = os.path.dirname(os.path.abspath(__file__))
    pkg = os.path.join(os.path.dirname(here), "mla-decode-kernels_amd")
    paths = [os.path.join(pkg, "python"), os.path.join(pkg, "bench"), os.path.dirname(here)]
    proc = subprocess.run([sys.executable, "-c", FIRST_CALL_UNDER_CAPTURE.format(paths=paths)],
                          capture_output=True, text=True, timeout=240)
    assert proc.returncode == 0 and "FIRST_CALL_UNDER_CAPTURE_OK" in proc.stdout, (
        proc.stdout[-2000:] + proc.stderr[-3000:])
