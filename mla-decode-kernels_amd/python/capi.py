"""ctypes view of the C ABI in include/gqa_decode.h (libgqa_decode_hip.so).

This is the binding a non-torch host would write over the same library; the
tests use it to drive the launchers directly -- caller-owned workspace,
error codes -- and to check that every declared entry point is exported.
Pointer arguments take integers (e.g. ``tensor.data_ptr()``); the stream is a
raw hipStream_t (``torch.cuda.current_stream().cuda_stream``).
"""

import ctypes
import os
import re

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_DIR, "lib", "libgqa_decode_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(_PKG_DIR), "include", "gqa_decode.h")
MLA_HEADER_PATH = os.path.join(os.path.dirname(_PKG_DIR), "include", "mla_decode.h")

HIP_SUCCESS = 0
HIP_ERROR_INVALID_VALUE = 1

_vp = ctypes.c_void_p
_i = ctypes.c_int
_LAUNCH_ARGS = [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, ctypes.c_float]

_lib = None


def declared_functions(header=None, prefix="gqa_decode_"):
    """Names of the functions a header of include/ declares (default:
    include/gqa_decode.h)."""
    with open(header or HEADER_PATH) as f:
        text = re.sub(r"/\*.*?\*/", "", f.read(), flags=re.S)
    pat = r"^\s*(?:GQA_DECODE_API\s+)?(?:int|size_t)\s+(" + prefix + r"\w+)\s*\("
    return sorted(set(re.findall(pat, text, flags=re.M)))


def declared_mla_functions():
    """Names of the functions include/mla_decode.h declares."""
    return declared_functions(MLA_HEADER_PATH, "mla_decode_")


def lib():
    """The in-tree library (LIB_PATH), loaded and bound once per process."""
    global _lib
    if _lib is None:
        _lib = bind(LIB_PATH)
    return _lib


def bind(path):
    """A build of the library at `path` with every entry point's signature set
    (a separate handle from lib(): tools load profiling builds this way)."""
    if not os.path.exists(path):
        raise OSError(f"{path} missing: run `python mla-decode-kernels_amd/build.py`")
    L = ctypes.CDLL(path)
    for name in ("gqa_decode_v0_launch", "gqa_decode_v1_launch"):
        fn = getattr(L, name)
        fn.argtypes = _LAUNCH_ARGS + [_vp]
        fn.restype = _i
    L.gqa_decode_v2_launch.argtypes = _LAUNCH_ARGS + [_i, _vp, _vp, _vp, _vp]
    L.gqa_decode_v2_launch.restype = _i
    L.gqa_decode_v2_partial_launch.argtypes = [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                               ctypes.c_float, _i, _vp, _vp, _vp, _vp]
    L.gqa_decode_v2_partial_launch.restype = _i
    L.gqa_decode_v2_merge_launch.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _vp]
    L.gqa_decode_v2_merge_launch.restype = _i
    L.gqa_decode_v2_workspace_bytes.argtypes = [_i, _i, _i]
    L.gqa_decode_v2_workspace_bytes.restype = ctypes.c_size_t
    L.gqa_decode_v2_fused_launch.argtypes = _LAUNCH_ARGS + [_i, _vp, ctypes.c_size_t, _vp]
    L.gqa_decode_v2_fused_launch.restype = _i
    L.gqa_decode_v2_fused_workspace_bytes.argtypes = [_i, _i, _i]
    L.gqa_decode_v2_fused_workspace_bytes.restype = ctypes.c_size_t
    L.gqa_decode_v2_fused_reset.argtypes = [_vp, ctypes.c_size_t, _i, _i, _i, _vp]
    L.gqa_decode_v2_fused_reset.restype = _i
    L.gqa_decode_pick_num_splits.argtypes = [_i, _i, _i, _i, _i, _i]
    L.gqa_decode_pick_num_splits.restype = _i
    L.gqa_decode_balanced_launch.argtypes = _LAUNCH_ARGS + [_i, _vp, ctypes.c_size_t, _vp]
    L.gqa_decode_balanced_launch.restype = _i
    L.gqa_decode_balanced_workspace_bytes.argtypes = [_i, _i, _i, _i]
    L.gqa_decode_balanced_workspace_bytes.restype = ctypes.c_size_t
    for name in ("gqa_decode_balanced_partial_launch", "gqa_decode_balanced_merge_launch"):
        fn = getattr(L, name)
        fn.argtypes = _LAUNCH_ARGS + [_i, _vp, ctypes.c_size_t, _vp]
        fn.restype = _i
    L.gqa_decode_balanced_launch_noalloc.argtypes = _LAUNCH_ARGS + [_i, _vp]
    L.gqa_decode_balanced_launch_noalloc.restype = _i
    L.gqa_decode_prefer_balanced.argtypes = [_i, _i, _i, _i, _i, _i]
    L.gqa_decode_prefer_balanced.restype = _i
    for fn in (L.mla_decode_launch, L.mla_decode_splitkv_launch, L.mla_decode_balanced_launch):
        fn.argtypes = [_vp] * 6 + [_i] * 5 + [ctypes.c_float, _i, _i, _vp, ctypes.c_size_t,
                                              _vp]
        fn.restype = _i
    L.mla_decode_combine_launch.argtypes = [_vp, ctypes.c_size_t, _vp, _vp, _i, _i, _i, _i,
                                            _vp]
    L.mla_decode_combine_launch.restype = _i
    L.mla_decode_balanced_workspace_bytes.argtypes = [_i] * 4
    L.mla_decode_balanced_workspace_bytes.restype = ctypes.c_size_t
    L.mla_decode_workspace_bytes.argtypes = [_i] * 4
    L.mla_decode_workspace_bytes.restype = ctypes.c_size_t
    L.mla_decode_pick_num_splits.argtypes = [_i] * 6
    L.mla_decode_pick_num_splits.restype = _i
    return L


def v0_launch(*args):
    return lib().gqa_decode_v0_launch(*args)


def v1_launch(*args):
    return lib().gqa_decode_v1_launch(*args)


def v2_launch(*args):
    return lib().gqa_decode_v2_launch(*args)


def v2_partial_launch(*args):
    return lib().gqa_decode_v2_partial_launch(*args)


def v2_merge_launch(*args):
    return lib().gqa_decode_v2_merge_launch(*args)


def workspace_bytes(B, Hq, num_splits):
    return lib().gqa_decode_v2_workspace_bytes(B, Hq, num_splits)


def v2_fused_launch(*args):
    return lib().gqa_decode_v2_fused_launch(*args)


def fused_workspace_bytes(B, Hq, num_splits):
    return lib().gqa_decode_v2_fused_workspace_bytes(B, Hq, num_splits)


def v2_fused_reset(*args):
    return lib().gqa_decode_v2_fused_reset(*args)


def pick_num_splits(B, Hq, Hkv, block_size, max_blocks, num_cus):
    return lib().gqa_decode_pick_num_splits(B, Hq, Hkv, block_size, max_blocks, num_cus)


def balanced_launch(*args):
    return lib().gqa_decode_balanced_launch(*args)


def balanced_workspace_bytes(B, Hq, Hkv, num_workgroups):
    return lib().gqa_decode_balanced_workspace_bytes(B, Hq, Hkv, num_workgroups)


def balanced_partial_launch(*args):
    return lib().gqa_decode_balanced_partial_launch(*args)


def balanced_merge_launch(*args):
    return lib().gqa_decode_balanced_merge_launch(*args)


def prefer_balanced(B, Hq, Hkv, block_size, max_blocks, num_cus):
    return lib().gqa_decode_prefer_balanced(B, Hq, Hkv, block_size, max_blocks, num_cus)


def mla_launch(*args):
    return lib().mla_decode_launch(*args)


def mla_splitkv_launch(*args):
    return lib().mla_decode_splitkv_launch(*args)


def mla_combine_launch(*args):
    return lib().mla_decode_combine_launch(*args)


def mla_balanced_launch(*args):
    return lib().mla_decode_balanced_launch(*args)


def mla_balanced_workspace_bytes(B, s_q, h_q, num_workgroups):
    return lib().mla_decode_balanced_workspace_bytes(B, s_q, h_q, num_workgroups)


def mla_workspace_bytes(B, s_q, h_q, num_splits):
    return lib().mla_decode_workspace_bytes(B, s_q, h_q, num_splits)


def mla_pick_num_splits(B, s_q, h_q, block_size, max_blocks, num_cus):
    return lib().mla_decode_pick_num_splits(B, s_q, h_q, block_size, max_blocks, num_cus)


def balanced_launch_noalloc(*args):
    """gqa_decode_balanced_launch_noalloc: the balanced launch on the library's
    own per-device scratch array (no workspace argument)."""
    return lib().gqa_decode_balanced_launch_noalloc(*args)


# GQA_DECODE_NOALLOC_SCRATCH_BYTES in include/gqa_decode.h.
NOALLOC_SCRATCH_BYTES = 32 << 20
