"""Synthetic paged-decode inputs and the speed-of-light arithmetic.

Counterpart of the reference's bench/common.py:16-72 and of the case builder
in tests/test_gqa_decode.py:27-69: seeded q/k/v, a shuffled physical block
pool, -1 padding past each request's blocks, and optional NaN poisoning of
every slot a kernel must not read (unallocated blocks and the tail slots of
each request's last block).
"""

import math

import numpy as np
import torch

D = 128
HBM_PEAK_BYTES_PER_S = 8.0e12  # MI355X HBM3E, AMD spec

# BASELINE.json configs 1..5.
CONFIGS = {
    "c1": dict(Hq=32, Hkv=8, B=1, S=512, bs=16, pool=64,
               desc="plumbing: B=1 S=512 block=16, 64-block pool (32 used)"),
    "c2": dict(Hq=32, Hkv=8, B=32, S=8192, bs=16, pool=16384,
               desc="representative: 32Q/8KV B=32 S=8192 block=16 (1 GiB KV)"),
    "c3": dict(Hq=32, Hkv=8, B=8, S=32768, bs=64, pool=4096,
               desc="long context: 32Q/8KV B=8 S=32768 block=64 (1 GiB KV)"),
    "c4": dict(Hq=64, Hkv=8, B=32, S=32768, bs=64, pool=16384,
               desc="wide GQA: 64Q/8KV B=32 S=32768 block=64 (4 GiB KV)"),
    "c5": dict(Hq=32, Hkv=8, B=128, S=None, S_max=32768, bs=16, pool_factor=1.25,
               desc="ragged: 32Q/8KV B=128 S~U[1,32768] block=16, pool 1.25x"),
}


def config_seq_lens(name, seed=0):
    """Per-request lengths of a config (the ragged one draws from a seeded CPU
    generator, so the lengths are identical on every machine)."""
    cfg = CONFIGS[name]
    if cfg["S"] is not None:
        return [cfg["S"]] * cfg["B"]
    g = torch.Generator().manual_seed(seed + 1)
    return torch.randint(1, cfg["S_max"] + 1, (cfg["B"],), generator=g).tolist()


def make_case(S_list, Hq, Hkv, bs, *, pool=None, pool_factor=None, seed=0, device="cuda",
              qkv_std=1.0, poison=False, max_blocks=None, shuffle=True):
    """Build (q, k_cache, v_cache, block_table, seq_lens) on `device`.

    q/k/v ~ qkv_std * N(0, 1) in bf16 from a seeded generator on `device`.
    The physical pool holds `pool` blocks (default ceil(pool_factor * needed),
    or exactly the needed count); block ids come from a seeded CPU permutation
    of the pool, request b taking the next ceil(S_b / bs) ids. Entries past a
    request's blocks are -1. With poison=True every unallocated block and every
    slot past S_b in a request's last block is NaN. shuffle=False hands out
    the pool in order (request b's blocks contiguous in memory).
    """
    B = len(S_list)
    n_blocks = [(int(s) + bs - 1) // bs for s in S_list]
    needed = sum(n_blocks)
    if pool is None:
        pool = math.ceil(needed * pool_factor) if pool_factor else needed
    if pool < needed:
        raise ValueError(f"pool of {pool} blocks < {needed} needed")
    if max_blocks is None:
        max_blocks = max(n_blocks) if n_blocks else 1

    gen = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn(B, Hq, D, device=device, generator=gen, dtype=torch.float32)
    q = (q * qkv_std).to(torch.bfloat16)
    k_cache = torch.empty(pool, bs, Hkv, D, device=device, dtype=torch.bfloat16)
    v_cache = torch.empty_like(k_cache)
    # Fill in slabs of blocks to bound the fp32 temporary.
    slab = max(1, (64 << 20) // (bs * Hkv * D))
    for cache in (k_cache, v_cache):
        for i in range(0, pool, slab):
            n = min(slab, pool - i)
            x = torch.randn(n, bs, Hkv, D, device=device, generator=gen, dtype=torch.float32)
            cache[i:i + n] = (x * qkv_std).to(torch.bfloat16)

    perm = (torch.randperm(pool, generator=torch.Generator().manual_seed(seed)) if shuffle
            else torch.arange(pool))
    block_table = torch.full((B, max_blocks), -1, dtype=torch.int32)
    used = torch.zeros(pool, dtype=torch.bool)
    off = 0
    for b in range(B):
        ids = perm[off:off + n_blocks[b]]
        block_table[b, :n_blocks[b]] = ids.to(torch.int32)
        used[ids] = True
        off += n_blocks[b]

    if poison:
        unused = (~used).nonzero().flatten().to(device)
        if unused.numel():
            k_cache.index_fill_(0, unused, float("nan"))
            v_cache.index_fill_(0, unused, float("nan"))
        for b in range(B):
            rem = int(S_list[b]) % bs
            if rem:
                last = int(block_table[b, n_blocks[b] - 1])
                k_cache[last, rem:] = float("nan")
                v_cache[last, rem:] = float("nan")

    seq_lens = torch.tensor([int(s) for s in S_list], dtype=torch.int32, device=device)
    return q, k_cache, v_cache, block_table.to(device), seq_lens


def make_config_case(name, seed=0, device="cuda", poison=False, shuffle=True):
    cfg = CONFIGS[name]
    S_list = config_seq_lens(name, seed)
    return make_case(S_list, cfg["Hq"], cfg["Hkv"], cfg["bs"], pool=cfg.get("pool"),
                     pool_factor=cfg.get("pool_factor"), seed=seed, device=device,
                     poison=poison, shuffle=shuffle)


# MLA decode workloads: the FlashMLA benchmark rows the reference keeps as its
# K2 baseline (docs/g0/flashmla_bench_raw.txt:4674-4719 of the reference):
# b=128, h_q=128, one latent head, d=576, dv=512, block 64, varlen lengths
# around s_k, s_q = 1 (plain decode) or 2 (two query tokens per request).
MLA_CONFIGS = {
    f"mla_{sk // 1024}k" + ("_sq2" if sq == 2 else ""): dict(B=128, s_q=sq, h_q=128, S_mean=sk,
                                                              bs=64, causal=False)
    for sq in (1, 2) for sk in (4096, 8192, 16384, 32768)
}


def mla_seq_lens(B, S_mean, seed=0, s_q=1):
    """FlashMLA's varlen draw, seeded: max(N(S_mean, S_mean / 2), s_q) per
    request, on a CPU generator so that every machine builds the same batch."""
    g = torch.Generator().manual_seed(seed + 7)
    x = torch.randn(B, generator=g, dtype=torch.float64) * (S_mean / 2) + S_mean
    return [max(int(v), s_q) for v in x.tolist()]


def make_mla_case(S_list, s_q, h_q, bs, *, pool=None, pool_factor=None, seed=0, device="cuda",
                  std=1.0, poison=False, shuffle=True):
    """(q [B, s_q, h_q, 576], kv_cache [pool, bs, 1, 576], block_table, seq_lens)
    on `device`, as make_case builds the GQA cases: seeded N(0, std^2) bf16,
    a shuffled pool, -1 past each request's blocks, and with poison=True NaN
    in every cache slot no request owns (including the tail of each last
    block)."""
    B = len(S_list)
    D = 576
    n_blocks = [(int(x) + bs - 1) // bs for x in S_list]
    needed = sum(n_blocks)
    if pool is None:
        pool = max(1, math.ceil(needed * pool_factor) if pool_factor else needed)
    gen = torch.Generator(device=device).manual_seed(seed)
    q = (torch.randn(B, s_q, h_q, D, device=device, generator=gen) * std).to(torch.bfloat16)
    kv = torch.empty(pool, bs, 1, D, device=device, dtype=torch.bfloat16)
    slab = max(1, (64 << 20) // (bs * D))
    for i in range(0, pool, slab):
        n = min(slab, pool - i)
        kv[i:i + n] = (torch.randn(n, bs, 1, D, device=device, generator=gen) * std).to(
            torch.bfloat16)
    perm = (torch.randperm(pool, generator=torch.Generator().manual_seed(seed)) if shuffle
            else torch.arange(pool))
    max_blocks = max(max(n_blocks), 1) if n_blocks else 1
    block_table = torch.full((B, max_blocks), -1, dtype=torch.int32)
    used = torch.zeros(pool, dtype=torch.bool)
    off = 0
    for b in range(B):
        ids = perm[off:off + n_blocks[b]]
        block_table[b, :n_blocks[b]] = ids.to(torch.int32)
        used[ids] = True
        off += n_blocks[b]
    if poison:
        unused = (~used).nonzero().flatten().to(device)
        if unused.numel():
            kv.index_fill_(0, unused, float("nan"))
        for b in range(B):
            rem = int(S_list[b]) % bs
            if rem:
                kv[int(block_table[b, n_blocks[b] - 1]), rem:] = float("nan")
    seq_lens = torch.tensor([int(x) for x in S_list], dtype=torch.int32, device=device)
    return q, kv, block_table.to(device), seq_lens


# FlashMLA's published H100 rows for these workloads (b=128, h_q=128, h_kv=1,
# block 64, varlen, not causal), ms per call: docs/g0/flashmla_bench_raw.txt
# of the reference, lines 4675-4697.
MLA_H100_MS = {"mla_4k": 0.274, "mla_8k": 0.504, "mla_16k": 0.962, "mla_32k": 1.873,
               "mla_4k_sq2": 0.425, "mla_8k_sq2": 0.805, "mla_16k_sq2": 1.565,
               "mla_32k_sq2": 3.096}


def mla_flops_bytes(seq_lens, s_q, h_q, d=576, dv=512):
    """FlashMLA's accounting of one decode step, the numbers its benchmark
    divides by the time: FLOPs of QK^T and PV over every query row and key
    (2 * s_q * h_q * sum(S) * (d + dv), no causal discount) and bytes of q,
    the latent rows once and the output (bf16)."""
    total = float(sum(max(int(x), 0) for x in seq_lens))
    B = len(seq_lens)
    flops = 2.0 * s_q * h_q * total * (d + dv)
    nbytes = (B * s_q * h_q * d + total * d + B * s_q * h_q * dv) * 2
    return flops, nbytes


def mla_host_case(case, batches):
    """Host (numpy) copy of the listed requests of an MLA case (q, kv_cache,
    block_table, seq_lens), their blocks compacted into a small pool with
    remapped ids."""
    q, kv, bt, sl = case
    batches = list(batches)
    bs = kv.shape[1]
    sl_h = sl.cpu().numpy()[batches]
    bt_h = bt.cpu().numpy()[batches]
    n = [(int(x) + bs - 1) // bs for x in sl_h]
    ids = np.concatenate([bt_h[i, :n[i]] for i in range(len(batches))]).astype(np.int64)
    new_bt = np.full((len(batches), max(max(n), 1)), -1, dtype=np.int32)
    off = 0
    for i in range(len(batches)):
        new_bt[i, :n[i]] = np.arange(off, off + n[i])
        off += n[i]
    pool = kv.index_select(0, torch.from_numpy(ids).to(kv.device))
    return bits(q[batches]), bits(pool), new_bt, sl_h.astype(np.int32)


def kv_bytes(S_list, Hkv):
    """Algorithmic K+V bytes of one decode step: sum_b S_b * Hkv * 128 * 2 * 2
    (bench/common.py:67-69 of the reference, per request)."""
    return sum(int(s) for s in S_list) * Hkv * D * 2 * 2


def sol_us(nbytes, peak=HBM_PEAK_BYTES_PER_S):
    """Speed-of-light time of streaming nbytes from HBM once, in microseconds."""
    return nbytes / peak * 1e6


def time_op(fn, warmup=10, runs=50):
    """Median time of fn() in milliseconds, HIP events on the current stream
    around each call (bench/common.py:49-64 of the reference)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    times = []
    for _ in range(runs):
        start.record()
        fn()
        end.record()
        end.synchronize()
        times.append(start.elapsed_time(end))
    times.sort()
    return times[len(times) // 2]


def bits(t):
    """bf16 device tensor -> uint16 numpy array of raw bits (on the host)."""
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def host_case(case, batches=None):
    """Host (numpy) copy of (q, k, v, block_table, seq_lens). With `batches`,
    only those requests are kept and their blocks are compacted into a small
    pool with remapped ids, so a large case can be checked on a subset."""
    q, k, v, bt, sl = case
    if batches is None:
        return bits(q), bits(k), bits(v), bt.cpu().numpy(), sl.cpu().numpy()
    batches = list(batches)
    bs = k.shape[1]
    sl_h = sl.cpu().numpy()[batches]
    bt_h = bt.cpu().numpy()[batches]
    n = [(int(s) + bs - 1) // bs for s in sl_h]
    ids = np.concatenate([bt_h[i, :n[i]] for i in range(len(batches))]).astype(np.int64)
    idx = torch.from_numpy(ids).to(k.device)
    new_bt = np.full((len(batches), max(n)), -1, dtype=np.int32)
    off = 0
    for i in range(len(batches)):
        new_bt[i, :n[i]] = np.arange(off, off + n[i])
        off += n[i]
    return (bits(q[batches]), bits(k.index_select(0, idx)), bits(v.index_select(0, idx)),
            new_bt, sl_h.astype(np.int32))


def gpu_clocks():
    """Current shader and memory clocks from the amdgpu sysfs DPM tables (the
    entry marked '*'); read directly so no helper process is started."""
    import glob
    import os

    out = {}
    for dev in sorted(glob.glob("/sys/class/drm/card*/device")):
        for key, fname in (("sclk", "pp_dpm_sclk"), ("mclk", "pp_dpm_mclk")):
            try:
                with open(os.path.join(dev, fname)) as f:
                    cur = [ln.split(":", 1)[1].strip(" *\n") for ln in f if ln.rstrip().endswith("*")]
                if cur:
                    out.setdefault(key, cur[0])
            except OSError:
                pass
        if out:
            break
    return out or "unavailable"


def torch_ref_fp32(q, k_cache, v_cache, block_table, seq_lens, scale, batches):
    """fp32 GQA decode of the listed requests, in torch on the tensors' device:
    gather the request's pages, fp32 scores, softmax, weighted V sum. A spot
    check for benchmark runs (the test suite checks against the CPU oracle)."""
    bs, Hkv, Dh = k_cache.shape[1:]
    Hq = q.shape[1]
    G = Hq // Hkv
    lens = seq_lens.tolist()
    outs = []
    for b in batches:
        S = int(lens[b])
        n = (S + bs - 1) // bs
        ids = block_table[b, :n].long()
        k = k_cache.index_select(0, ids).view(n * bs, Hkv, Dh)[:S].float()
        v = v_cache.index_select(0, ids).view(n * bs, Hkv, Dh)[:S].float()
        k = k.permute(1, 2, 0).contiguous()                 # [Hkv, D, S]
        v = v.permute(1, 0, 2).contiguous()                 # [Hkv, S, D]
        qb = q[b].float().view(Hkv, G, Dh)
        p = torch.softmax(torch.bmm(qb, k) * scale, dim=-1)  # [Hkv, G, S]
        outs.append(torch.bmm(p, v).reshape(Hq, Dh))
    return torch.stack(outs)


def spot_check(fn, case, scale, label="kernel", nb=2, tol=2e-2):
    """Run fn(*case, scale) once and compare its first min(nb, B) requests with
    torch_ref_fp32 (bench/common.py:75-89 of the reference). Returns the
    max-abs error; raises AssertionError beyond atol = rtol = tol."""
    nb = min(nb, case[0].shape[0])
    out = fn(*case, scale)
    torch.cuda.synchronize()
    ref = torch_ref_fp32(*case, scale, range(nb))
    got = out[:nb].float()
    max_abs = (got - ref).abs().max().item()
    assert torch.allclose(got, ref, atol=tol, rtol=tol), (
        f"{label} spot check failed on first {nb} requests: max-abs={max_abs:.4e}")
    return max_abs


def time_ops_two_pass(fns, warmup=10, runs=50):
    """Median time in milliseconds of each zero-argument callable in `fns`
    (name -> fn), each measured as time_op measures it (the reference's
    method: back-to-back calls, events around each, synchronize after each),
    in two passes over the callables, the second in reverse order; each keeps
    the lower of its two medians. Slow drifts within a run (clocks, power
    state) then cannot favour whichever callable happens to be measured last."""
    names = list(fns)
    best = {}
    for order in (names, names[::-1]):
        for name in order:
            t = time_op(fns[name], warmup, runs)
            best[name] = min(best.get(name, t), t)
    return best
