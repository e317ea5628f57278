"""Build recipe for the gfx950 GQA decode library and its PyTorch extension.

    python mla-decode-kernels_amd/build.py            # kernels + extension
    python mla-decode-kernels_amd/build.py --no-ext   # kernel library only
    python mla-decode-kernels_amd/build.py --variant NAME --define MACRO=VALUE ...
        # an experiment build of the kernel library with compile-time
        # switches, into _build/NAME/ (git-ignored; for bench.py --lib)

Products (in-tree, git-ignored, shipped with the source tree):
  lib/libgqa_decode_hip.so   hipcc --offload-arch=gfx950: every kernel + the C ABI
                             (+ .sources.json: the source hashes it was built
                             from, python/provenance.py)
  lib/gqa_decode_ext*.so     g++: host-only torch operator layer linking the above
  lib/libgqa_stream_probe.so hipcc: the streaming-read probe bench.py measures
                             the bandwidth ceiling with (not on the decode path)
  lib/libissue_probe.so      hipcc: MFMA / VALU / LDS issue-rate probes and the
                             lane-swap probe (bench/issue_probe.py,
                             tests/test_profile_tools.py; not on the decode path)
  _build/phase/libgqa_decode_hip.so
                             the kernel library built with MLA_PHASE_TIMING=1
                             (bench/mla_phases.py; not on the decode path)

The extension is compiled as plain C++ (no .cu/.hip source, so torch's
hipify pass never runs); it reaches the GPU only through the C ABI.
"""

import argparse
import os
import shutil
import subprocess
import sys
import sysconfig
import time
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_ROOT = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_DIR = os.path.join(PKG_DIR, "lib")
INCLUDE = os.path.join(REPO_ROOT, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

KERNEL_LIB = os.path.join(LIB_DIR, "libgqa_decode_hip.so")
# The MLA decode's phase-timing build (bench/mla_phases.py reads its table).
PHASE_LIB = os.path.join(PKG_DIR, "_build", "phase", "libgqa_decode_hip.so")
PHASE_DEFINES = ["MLA_PHASE_TIMING=1"]
OBJ_DIR = os.path.join(PKG_DIR, "_build", "obj")  # objects: not shipped to GPU runs
PROBE_LIB = os.path.join(LIB_DIR, "libgqa_stream_probe.so")
ISSUE_PROBE_LIB = os.path.join(LIB_DIR, "libissue_probe.so")
HIP_SOURCES = ["gqa_decode_v0.hip", "gqa_decode_split.hip", "gqa_decode_mfma.hip",
               "gqa_decode_balanced.hip", "mla_decode.hip"]
# Packed fp32 VALU ops are disabled for all device code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd, cwd=None):
    t0 = time.time()
    proc = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the device-only feature flag; drop that note.
    out = "\n".join(
        ln for ln in proc.stdout.splitlines()
        if "packed-fp32-ops' is not a recognized feature" not in ln
    )
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)
    return time.time() - t0


def build_kernels(out=KERNEL_LIB, defines=()):
    """hipcc every HIP source to an object (in parallel), then link them into
    the shared library `out`, with the source hashes next to it."""
    os.makedirs(os.path.dirname(out), exist_ok=True)
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    flags = [f"-D{d}" for d in defines]
    tag = os.path.relpath(out, PKG_DIR).replace(os.sep, "_")
    objdir = os.path.join(OBJ_DIR, tag)
    os.makedirs(objdir, exist_ok=True)
    t0 = time.time()
    objs = [os.path.join(objdir, os.path.splitext(src)[0] + ".o") for src in HIP_SOURCES]
    with ThreadPoolExecutor(max_workers=len(HIP_SOURCES)) as pool:
        list(pool.map(lambda so: _run([hipcc, *HIP_FLAGS, *flags, f"-I{INCLUDE}", "-c",
                                       os.path.join(CSRC, so[0]), "-o", so[1]]),
                      zip(HIP_SOURCES, objs)))
    tmp = out + ".tmp"
    _run([hipcc, *HIP_FLAGS, "-shared", *objs, "-o", tmp])
    os.replace(tmp, out)
    # The source hashes this library was built from (results carry them).
    sys.path.insert(0, os.path.join(PKG_DIR, "python"))
    import provenance
    provenance.write_sidecar(out, defines)
    print(f"built {os.path.relpath(out, REPO_ROOT)} in {time.time() - t0:.1f}s")
    return out


def build_probe(src="stream_probe.hip", lib=PROBE_LIB):
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    tmp = lib + ".tmp"
    dt = _run([hipcc, *HIP_FLAGS, "-shared", os.path.join(CSRC, src), "-o", tmp])
    os.replace(tmp, lib)
    print(f"built {os.path.relpath(lib, REPO_ROOT)} in {dt:.1f}s")
    return lib


def ext_filename():
    return "gqa_decode_ext" + sysconfig.get_config_var("EXT_SUFFIX")


def build_extension():
    import torch
    from torch.utils import cpp_extension

    if not os.path.exists(KERNEL_LIB):
        raise RuntimeError("kernel library missing; build it first")
    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = cpp_extension.include_paths() + [INCLUDE, os.path.join(ROCM, "include"),
                                            sysconfig.get_paths()["include"]]
    out = os.path.join(LIB_DIR, ext_filename())
    tmp = out + ".tmp"
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-w",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_API_INCLUDE_EXTENSION_H",
        "-DTORCH_EXTENSION_NAME=gqa_decode_ext", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        *[f"-I{i}" for i in incs],
        os.path.join(PKG_DIR, "python", "gqa_decode_ext.cpp"),
        "-o", tmp,
        f"-L{LIB_DIR}", "-lgqa_decode_hip", "-Wl,-rpath,$ORIGIN",
        f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
        f"-Wl,-rpath,{torch_lib}",
        f"-L{os.path.join(ROCM, 'lib')}", "-lamdhip64",
    ]
    dt = _run(cmd)
    os.replace(tmp, out)
    print(f"built {os.path.relpath(out, REPO_ROOT)} in {dt:.1f}s")
    return out


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--no-ext", action="store_true", help="build the kernel library only")
    ap.add_argument("--variant", default=None,
                    help="build only the kernel library, into _build/VARIANT/")
    ap.add_argument("--define", action="append", default=[], metavar="MACRO[=VALUE]",
                    help="compile-time switch for a --variant build (e.g. GQA_MFMA_MIN_GROUP=17)")
    args = ap.parse_args(argv)
    if shutil.which(os.path.join(ROCM, "bin", "hipcc")) is None:
        sys.exit(f"hipcc not found under {ROCM}")
    if args.define and not args.variant:
        ap.error("--define needs --variant (the in-tree library is built as shipped)")
    if args.variant:
        build_kernels(os.path.join(PKG_DIR, "_build", args.variant, "libgqa_decode_hip.so"),
                      args.define)
        return
    build_kernels()
    build_kernels(PHASE_LIB, PHASE_DEFINES)
    build_probe()
    build_probe("issue_probe.hip", ISSUE_PROBE_LIB)
    if not args.no_ext:
        build_extension()


if __name__ == "__main__":
    main()
