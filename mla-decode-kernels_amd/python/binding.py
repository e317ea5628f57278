"""Python surface of the gfx950 GQA decode kernels.

Mirrors the reference's python/binding.py:25-31: ``gqa_decode_v0``,
``gqa_decode_v1``, ``gqa_decode_v2`` (num_splits defaults to 8; 0 selects the
CU-count heuristic) and the ``KERNELS`` dict. The reference JIT-compiles its
CUDA sources on import (python/binding.py:11-23); this package loads the
extension that ``mla-decode-kernels_amd/build.py`` built in-tree, and raises
ImportError when it is missing -- there is no fallback implementation.
"""

import glob
import importlib.util
import os

import torch  # noqa: F401  (loads libtorch / libc10_hip before the extension)

_LIB_DIR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "lib")


def _load_extension():
    paths = sorted(glob.glob(os.path.join(_LIB_DIR, "gqa_decode_ext*.so")))
    if not paths:
        raise ImportError(
            f"gqa_decode_ext not built in {_LIB_DIR}; run "
            "`python mla-decode-kernels_amd/build.py` (or __graft_entry__.build())"
        )
    spec = importlib.util.spec_from_file_location("gqa_decode_ext", paths[0])
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


_ext = _load_extension()
EXTENSION_PATH = _ext.__file__

gqa_decode_v0 = _ext.gqa_decode_v0
gqa_decode_v1 = _ext.gqa_decode_v1
gqa_decode_v2 = _ext.gqa_decode_v2
num_splits_heuristic = _ext.num_splits_heuristic
# Beyond the reference: the token-balanced split-KV launch, and the rule the
# v2 op's num_splits=0 uses to choose it.
gqa_decode_balanced = _ext.gqa_decode_balanced
prefer_balanced = _ext.prefer_balanced
# What gqa_decode_v2(..., num_splits=0) runs: 0 = the balanced launch, else the
# split count.
automatic_choice = _ext.automatic_choice

# "v2" runs with its default num_splits=8; pass num_splits explicitly via
# gqa_decode_v2 to override (0 = heuristic).
KERNELS = {"v0": gqa_decode_v0, "v1": gqa_decode_v1, "v2": gqa_decode_v2}
