"""Where the MLA decode's waves spend their cycles: the phase table of a
profiling build of the kernel library.

    python mla-decode-kernels_amd/build.py --variant phase --define MLA_PHASE_TIMING=1
    python mla-decode-kernels_amd/bench/mla_phases.py --config mla_4k

The profiling build stamps the shader clock (s_memtime) at the phase
boundaries of every full tile interval and of every piece, per wave, and adds
the cycles up on the device (csrc/mla_decode.hip, MLA_PHASE_TIMING). This
script runs the token-balanced launch of a FlashMLA benchmark row through the
C ABI of that build, reads the table back and prints, as markdown:
  - the shader clock over the split kernel (s_memtime against the 100 MHz
    s_memrealtime);
  - cycles per full interval and wave, by phase, for the PV-first waves
    (0-3: copies, PV of the previous tile, QK^T, softmax, barrier) and the
    QK-first waves (4-7: QK^T, softmax, PV, barrier);
  - cycles per launch and wave outside the full intervals: Q loads, the
    prologue (first tiles), the first and last intervals of each piece, the
    restart vote and the epilogue (stores).
The stamps cost a few percent of the step; the shipped library has none.
"""

import argparse
import ctypes
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.dirname(HERE)
for p in (os.path.join(PKG_DIR, "python"), HERE):
    if p not in sys.path:
        sys.path.insert(0, p)

COLS = ["copies", "first (PV)", "QK^T", "softmax", "second (PV)", "barrier", "intervals",
        "Q load", "prologue", "first interval", "last interval", "vote", "epilogue", "pieces",
        "kernel", "kernel realtime"]
ROWS = 2048


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--config", default="mla_4k")
    ap.add_argument("--lib", default=os.path.join(PKG_DIR, "_build", "phase", "libgqa_decode_hip.so"))
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--seed", type=int, default=0)
    args = ap.parse_args(argv)

    import numpy as np
    import torch

    import capi
    import cases

    # Its own handle on the profiling build: the launches below must run the
    # build whose table is read back, whatever library this process loaded
    # before (capi.lib(), the torch extension).
    raw = capi.bind(os.path.abspath(args.lib))
    if not hasattr(raw, "mla_decode_phase_table"):
        sys.exit(f"{args.lib} is not a MLA_PHASE_TIMING build")
    raw.mla_decode_phase_table.argtypes = [ctypes.c_void_p, ctypes.c_int]
    dev = torch.device("cuda", 0)
    cfg = cases.MLA_CONFIGS[args.config]
    B, s_q, h_q, bs = cfg["B"], cfg["s_q"], cfg["h_q"], cfg["bs"]
    S_list = cases.mla_seq_lens(B, cfg["S_mean"], args.seed, s_q)
    q, kv, bt, sl = cases.make_mla_case(S_list, s_q, h_q, bs, seed=args.seed, device=dev)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    out = torch.empty(B, s_q, h_q, 512, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(B, h_q, s_q, dtype=torch.float32, device=dev)
    wsb = raw.mla_decode_balanced_workspace_bytes(B, s_q, h_q, cus)
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=dev)
    largs = (q.data_ptr(), kv.data_ptr(), bt.data_ptr(), sl.data_ptr(), out.data_ptr(),
             lse.data_ptr(), B, s_q, h_q, bs, bt.shape[1], 576 ** -0.5, 0, cus, ws.data_ptr(), wsb,
             torch.cuda.current_stream().cuda_stream)

    def step():
        if raw.mla_decode_balanced_launch(*largs) != 0:
            raise RuntimeError("mla_decode_balanced_launch failed")

    for _ in range(20):
        step()
    torch.cuda.synchronize()
    if raw.mla_decode_phase_table(None, 1) != 0:
        raise RuntimeError("phase table reset failed")
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ev[0].record()
    for _ in range(args.steps):
        step()
    ev[1].record()
    torch.cuda.synchronize()
    step_us = ev[0].elapsed_time(ev[1]) * 1e3 / args.steps
    buf = np.zeros((ROWS, len(COLS)), dtype=np.uint64)
    if raw.mla_decode_phase_table(ctypes.c_void_p(buf.ctypes.data), 0) != 0:
        raise RuntimeError("phase table read failed")
    t = buf.astype(np.float64).reshape(-1, 8, len(COLS))[:min(cus, 256)]
    waves = t.shape[0] * 8 * args.steps  # wave launches recorded
    kern = t[:, :, COLS.index("kernel")].sum() / waves
    mhz = t[:, :, COLS.index("kernel")].sum() / t[:, :, COLS.index("kernel realtime")].sum() * 100

    print(f"# MLA decode phase table — {args.config} (token-balanced launch, {cus} CUs)\n")
    print(f"Step (profiling build, events): {step_us:.1f} us. Split kernel per wave: "
          f"{kern:.0f} cycles at {mhz:.0f} MHz ({kern / mhz:.1f} us).\n")
    print("Cycles per full interval and wave:\n")
    print("| waves | copies | first (PV) | QK^T | softmax | second (PV) | barrier | total |")
    print("|---|---|---|---|---|---|---|---|")
    for name, sel in (("PV-first 0-3", slice(0, 4)), ("QK-first 4-7", slice(4, 8))):
        x = t[:, sel, :]
        n = x[:, :, COLS.index("intervals")].sum()
        vals = [x[:, :, k].sum() / n for k in range(6)]
        print(f"| {name} | " + " | ".join(f"{v:.0f}" for v in vals) + f" | {sum(vals):.0f} |")
    print("\nCycles per launch and wave (all waves):\n")
    print("| full intervals | Q load | prologue | first interval | last interval | vote | "
          "epilogue | pieces per wave |")
    print("|---|---|---|---|---|---|---|---|")
    ints = t[:, :, :6].sum() / waves
    rest = [t[:, :, COLS.index(c)].sum() / waves for c in
            ("Q load", "prologue", "first interval", "last interval", "vote", "epilogue")]
    pieces = t[:, :, COLS.index("pieces")].sum() / waves
    print(f"| {ints:.0f} ({ints / kern:.0%}) | " + " | ".join(f"{v:.0f}" for v in rest) +
          f" | {pieces:.2f} |")
    print(f"\nFull intervals per wave per launch: "
          f"{t[:, :, COLS.index('intervals')].sum() / waves:.1f}.")
    return 0


if __name__ == "__main__":
    sys.exit(main())
