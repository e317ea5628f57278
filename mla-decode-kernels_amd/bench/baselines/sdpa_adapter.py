"""Vendor-library baseline: torch's scaled_dot_product_attention on ROCm.

This image ships no paged-decode library for ROCm (no FlashInfer, vLLM, aiter
or flash-attn packages); the attention kernels that are installed are the ones
torch dispatches to through AOTriton (its flash and memory-efficient
backends). This adapter runs one of those on the same inputs, in the role the
reference gives FlashInfer (bench/baselines/flashinfer_adapter.py:54-66):

* plan (untimed, once per batch): convert the page table to CSR pages
  (``block_table_to_paged``) and gather each request's pages into a
  contiguous ``[B, Hkv, S, 128]`` K and V -- the library has no paged input,
  so paging is resolved here, as FlashInfer's plan() resolves its schedule;
* run (timed): one SDPA call. The q-head group of each kv-head is folded into
  the query axis (q ``[B, Hq, 128]`` viewed as ``[B, Hkv, G, 128]``, no
  mask), which is exactly GQA decode with ``kv = h / G`` and reads every K/V
  row once, as a decode kernel does.

The timing contract is the reference's run()-only rule
(docs/decisions/k1-007-baseline-fairness.md:5-13). The math backend is never
allowed (it would materialise the score matrix through batched bf16
products): if neither AOTriton backend accepts a shape the call raises.
A batch of uniform length runs as one call; a ragged batch (the reference's
test cases) runs one call per request, so only uniform batches are timed.
"""

import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from .paged import block_table_to_paged

BACKENDS = {
    "flash": [SDPBackend.FLASH_ATTENTION],
    "efficient": [SDPBackend.EFFICIENT_ATTENTION],
    "auto": [SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION],
}


def gather_contiguous(cache, indices, S):
    """Paged cache [num_blocks, bs, Hkv, D] + the CSR page ids of R requests
    of uniform length S (R * ceil(S/bs) ids) -> contiguous [R, Hkv, S, D]."""
    bs, Hkv, D = cache.shape[1:]
    n = (S + bs - 1) // bs
    R = indices.numel() // n
    rows = cache.index_select(0, indices.to(torch.int64))      # [R*n, bs, Hkv, D]
    rows = rows.view(R, n * bs, Hkv, D)[:, :S]
    return rows.permute(0, 2, 1, 3).contiguous()


def make_sdpa_runner(q, k_cache, v_cache, block_table, seq_lens, scale, backend="auto"):
    """Plan now (untimed); return a zero-argument callable that only runs SDPA
    and returns out [B, Hq, 128] bf16."""
    B, Hq, D = q.shape
    bs, Hkv = k_cache.shape[1], k_cache.shape[2]
    if Hq % Hkv:
        raise ValueError("Hq must be a multiple of Hkv")
    lens = [int(s) for s in seq_lens.tolist()]
    if min(lens, default=1) < 1:
        raise ValueError("seq_lens must be >= 1")
    indptr, indices, _ = block_table_to_paged(block_table, seq_lens, bs)
    qg = q.contiguous().view(B, Hkv, Hq // Hkv, D)
    backends = BACKENDS[backend]
    if B == 0:
        return lambda: torch.empty_like(q)

    if len(set(lens)) == 1:
        S = lens[0]
        k = gather_contiguous(k_cache, indices, S)
        v = gather_contiguous(v_cache, indices, S)

        def run():
            with sdpa_kernel(backends):
                out = F.scaled_dot_product_attention(qg, k, v, scale=scale)
            return out.view(B, Hq, D)

        return run

    ptr = indptr.tolist()
    kv = [(gather_contiguous(k_cache, indices[ptr[b]:ptr[b + 1]], lens[b]),
           gather_contiguous(v_cache, indices[ptr[b]:ptr[b + 1]], lens[b])) for b in range(B)]

    def run_ragged():
        out = torch.empty_like(q)
        with sdpa_kernel(backends):
            for b, (k, v) in enumerate(kv):
                o = F.scaled_dot_product_attention(qg[b:b + 1], k, v, scale=scale)
                out[b] = o.view(Hq, D)
        return out

    return run_ragged


def sdpa_decode(q, k_cache, v_cache, block_table, seq_lens, scale, backend="auto"):
    """One-shot plan + run."""
    return make_sdpa_runner(q, k_cache, v_cache, block_table, seq_lens, scale, backend)()
