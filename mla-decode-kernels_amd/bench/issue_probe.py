"""MFMA, VALU and LDS issue rates of one MI355X CU, as markdown: the
measurements behind the MLA decode's wave layout (csrc/issue_probe.hip,
lib/libissue_probe.so, built by build.py).

    python mla-decode-kernels_amd/bench/issue_probe.py [--iters N]

One workgroup per CU runs each probe; rates are per chip (MFMA: dense bf16
FLOP/s of v_mfma_f32_16x16x32_bf16) or per CU (LDS: bytes of ds_read_b128 per
ns). Clock: the shader clock of wave 0 over its loop.
"""

import argparse
import ctypes
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(os.path.dirname(HERE), "lib", "libissue_probe.so")


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--iters", type=int, default=20000)
    args = ap.parse_args(argv)
    import torch

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    lib = ctypes.CDLL(LIB)
    lib.issue_probe_run.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    rows = (ctypes.c_double * (6 * 64))()
    n = lib.issue_probe_run(rows, 64, cus, args.iters)
    if n < 0:
        raise RuntimeError("issue_probe_run failed")
    print(f"# Issue-rate probes ({cus} CUs, {args.iters} iterations per wave)\n")
    print("| probe | waves per SIMD | MFMA chains | FMAs per iteration | ns per iteration "
          "and wave | dense bf16 TFLOP/s | clock MHz |")
    print("|---|---|---|---|---|---|---|")
    lds = []
    for i in range(n):
        kind, p1, p2, thr, ms, mhz = rows[6 * i:6 * i + 6]
        if kind == 1:
            lds.append((int(p1), int(thr), ms))
            continue
        waves = cus * thr / 64
        tf = waves * args.iters * p1 * 16384 / (ms * 1e-3) / 1e12 if p1 else 0.0
        name = "mfma" if p2 == 0 else ("valu" if p1 == 0 else "mfma + valu")
        print(f"| {name} | {int(thr) // 256} | {int(p1)} | {int(p2)} | "
              f"{ms * 1e6 / args.iters:.2f} | {tf:.0f} | {mhz:.0f} |")
    print("\n| LDS probe | waves per CU | reads in flight per wave | bytes per ns per CU |")
    print("|---|---|---|---|")
    for nr, thr, ms in lds:
        b = cus * (thr / 64) * args.iters * nr * 1024
        print(f"| ds_read_b128 | {thr // 64} | {nr} | {b / cus / (ms * 1e6):.1f} |")
    return 0


if __name__ == "__main__":
    sys.exit(main())
