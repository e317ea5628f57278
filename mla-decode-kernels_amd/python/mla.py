"""FlashMLA-style Python surface of the gfx950 MLA decode kernel.

The reference's K2 roadmap item (README.md:405-408 of the reference) names
FlashMLA, pinned at 15f13e5 (docs/g0/flashmla_sha.txt), as its baseline; its
Python calls are the interface a caller of the reference's K2 would code
against, so this module mirrors their names, argument order and meaning:

    tile_scheduler_metadata, num_splits = get_mla_metadata(
        cache_seqlens, s_q * h_q // h_kv, h_kv)
    out, softmax_lse = flash_mla_with_kvcache(
        q, k_cache, block_table, cache_seqlens, head_dim_v,
        tile_scheduler_metadata, num_splits, softmax_scale=None, causal=False)

q [b, s_q, h_q, 576] bf16, k_cache [num_blocks, block_size, 1, 576] bf16,
block_table [b, max_blocks] int32, cache_seqlens [b] int32 -> out
[b, s_q, h_q, 512] bf16, softmax_lse [b, h_q, s_q] fp32 (natural log).
FlashMLA's metadata drives its persistent scheduler; here it selects the
launch: the token-balanced one (equal shares of the batch's tiles per CU,
planned on the device) by default, or N fixed splits per request. num_splits
is the per-request cumulative count of partial results [b + 1], as in
FlashMLA.
The kernel is reached only through include/mla_decode.h (capi); there is no
CPU fallback.
"""

import math

import torch

import capi

HEAD_DIM = 576
HEAD_DIM_V = 512


def _cu_count(device):
    return torch.cuda.get_device_properties(device).multi_processor_count


def get_mla_metadata(cache_seqlens, num_heads_per_head_k, num_heads_k=1, max_seqlen=None,
                     block_size=64, num_splits=None):
    """The launch plan for a batch: (tile_scheduler_metadata, num_splits).

    tile_scheduler_metadata is a host int32 tensor [1, 8] (read on the host,
    so a decode step costs no device synchronisation): [0, 0] = 0 selects the
    token-balanced launch with [0, 1] workgroups (the device's CU count);
    [0, 0] = N > 0 selects N fixed splits per request. num_splits is, as in
    FlashMLA, the cumulative count of partial results per request ([b + 1]
    int32 on cache_seqlens' device), computed on the device for the balanced
    plan. num_heads_per_head_k is s_q * h_q // h_kv; num_heads_k must be 1.
    Passing num_splits=N asks for the fixed-split plan (max_seqlen bounds the
    longest request for the split heuristic when N is 0)."""
    if num_heads_k != 1:
        raise ValueError("MLA decode supports one latent kv head (num_heads_k == 1)")
    if cache_seqlens.dtype != torch.int32 or cache_seqlens.dim() != 1:
        raise ValueError("cache_seqlens must be a 1-D int32 tensor")
    b = cache_seqlens.numel()
    dev = cache_seqlens.device
    cus = _cu_count(dev) if dev.type == "cuda" else 0
    meta = torch.zeros(1, 8, dtype=torch.int32)
    if num_splits is not None:
        ns = int(num_splits)
        if ns == 0:
            if max_seqlen is None:
                max_seqlen = int(cache_seqlens.max().item()) if b else 0
            max_blocks = max(1, math.ceil(max(int(max_seqlen), 1) / block_size))
            ns = capi.mla_pick_num_splits(max(b, 1), 1, int(num_heads_per_head_k), block_size,
                                          max_blocks, cus)
        if ns <= 0:
            raise ValueError("get_mla_metadata: invalid arguments")
        meta[0, 0] = ns
        return meta, torch.arange(b + 1, dtype=torch.int32, device=dev) * ns
    rows = int(num_heads_per_head_k)
    groups = max(1, -(-rows // 128))
    nwg = cus or 256
    meta[0, 1] = nwg
    # Pieces per request under the balanced plan (share w of n takes tiles
    # [w T / n, (w + 1) T / n) of the request-ordered 32-token tiles).
    n_share = max(1, nwg // groups)
    tiles = (cache_seqlens.clamp(min=0).to(torch.int64) + 31) // 32
    pre = torch.cumsum(tiles, 0)
    p1, p0 = pre, pre - tiles
    T = pre[-1:].clamp(min=1) if b else torch.ones(1, dtype=torch.int64, device=dev)
    n = torch.minimum(torch.full_like(T, n_share), T)
    w_lo = ((p0 + 1) * n - 1) // T
    w_hi = (p1 * n - 1) // T
    pieces = torch.where(tiles > 0, w_hi - w_lo + 1, torch.zeros_like(tiles))
    splits = torch.zeros(b + 1, dtype=torch.int32, device=dev)
    splits[1:] = torch.cumsum(pieces, 0).to(torch.int32)
    return meta, splits


def flash_mla_with_kvcache(q, k_cache, block_table, cache_seqlens, head_dim_v,
                           tile_scheduler_metadata=None, num_splits=None, softmax_scale=None,
                           causal=False):
    """MLA absorbed-path decode over a paged latent cache; returns
    (out, softmax_lse). softmax_scale defaults to 576 ** -0.5."""
    if q.dtype != torch.bfloat16 or k_cache.dtype != torch.bfloat16:
        raise ValueError("q and k_cache must be bfloat16")
    if q.dim() != 4 or q.shape[-1] != HEAD_DIM or not q.is_contiguous():
        raise ValueError("q must be a contiguous [b, s_q, h_q, 576] tensor")
    if k_cache.dim() != 4 or k_cache.shape[-1] != HEAD_DIM or k_cache.shape[2] != 1 or \
            not k_cache.is_contiguous():
        raise ValueError("k_cache must be a contiguous [num_blocks, block_size, 1, 576] tensor")
    if head_dim_v != HEAD_DIM_V:
        raise ValueError("head_dim_v must be 512")
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or \
            not block_table.is_contiguous():
        raise ValueError("block_table must be a contiguous 2-D int32 tensor")
    if cache_seqlens.dtype != torch.int32 or cache_seqlens.dim() != 1:
        raise ValueError("cache_seqlens must be a 1-D int32 tensor")
    b, s_q, h_q, _ = q.shape
    if block_table.shape[0] != b or cache_seqlens.shape[0] != b:
        raise ValueError("batch sizes of q, block_table and cache_seqlens differ")
    for t in (k_cache, block_table, cache_seqlens):
        if t.device != q.device:
            raise ValueError("all tensors must be on the same device")
    bs = k_cache.shape[1]
    max_blocks = block_table.shape[1]
    ns = 0
    nwg = 0
    if tile_scheduler_metadata is not None:
        if tile_scheduler_metadata.device.type != "cpu":
            raise ValueError("tile_scheduler_metadata must be the host tensor get_mla_metadata "
                             "returns")
        ns = int(tile_scheduler_metadata[0, 0])
        nwg = int(tile_scheduler_metadata[0, 1])
    scale = HEAD_DIM ** -0.5 if softmax_scale is None else float(softmax_scale)
    out = torch.empty(b, s_q, h_q, HEAD_DIM_V, dtype=torch.bfloat16, device=q.device)
    lse = torch.empty(b, h_q, s_q, dtype=torch.float32, device=q.device)
    stream = torch.cuda.current_stream(q.device).cuda_stream
    ptrs = (q.data_ptr(), k_cache.data_ptr(), block_table.data_ptr(), cache_seqlens.data_ptr(),
            out.data_ptr(), lse.data_ptr(), b, s_q, h_q, bs, max_blocks, scale,
            int(bool(causal)))
    if ns > 0:
        wsb = capi.mla_workspace_bytes(b, s_q, h_q, ns)
        ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=q.device)
        rc = capi.mla_launch(*ptrs, ns, ws.data_ptr(), wsb, stream)
    else:
        nwg = nwg or _cu_count(q.device)
        wsb = capi.mla_balanced_workspace_bytes(b, s_q, h_q, nwg)
        ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=q.device)
        rc = capi.mla_balanced_launch(*ptrs, nwg, ws.data_ptr(), wsb, stream)
    if rc != 0:
        raise RuntimeError(f"MLA decode launch failed with HIP error {rc}")
    return out, lse
