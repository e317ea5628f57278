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
FlashMLA's metadata drives its own persistent scheduler; here it carries the
split count of the split-KV launch (tile_scheduler_metadata[0, 0]) and
num_splits is the per-request cumulative split count [b + 1], as in FlashMLA.
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
                     block_size=64):
    """Split count for a batch: (tile_scheduler_metadata [1, 8] int32,
    num_splits [b + 1] int32), both on cache_seqlens' device.

    num_heads_per_head_k is s_q * h_q // h_kv, as FlashMLA takes it; num_heads_k
    must be 1. max_seqlen bounds the longest request (default: read from
    cache_seqlens, one device-to-host copy; pass it to avoid the sync)."""
    if num_heads_k != 1:
        raise ValueError("MLA decode supports one latent kv head (num_heads_k == 1)")
    if cache_seqlens.dtype != torch.int32 or cache_seqlens.dim() != 1:
        raise ValueError("cache_seqlens must be a 1-D int32 tensor")
    b = cache_seqlens.numel()
    if max_seqlen is None:
        max_seqlen = int(cache_seqlens.max().item()) if b else 0
    max_blocks = max(1, math.ceil(max(int(max_seqlen), 1) / block_size))
    dev = cache_seqlens.device
    ns = capi.mla_pick_num_splits(max(b, 1), 1, int(num_heads_per_head_k), block_size, max_blocks,
                                  _cu_count(dev) if dev.type == "cuda" else 0)
    if ns <= 0:
        raise ValueError("get_mla_metadata: invalid arguments")
    meta = torch.zeros(1, 8, dtype=torch.int32, device=dev)
    meta[0, 0] = ns
    splits = torch.arange(b + 1, dtype=torch.int32, device=dev) * ns
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
    if tile_scheduler_metadata is not None:
        ns = int(tile_scheduler_metadata[0, 0].item())
    else:
        ns = capi.mla_pick_num_splits(max(b, 1), s_q, h_q, bs, max_blocks, _cu_count(q.device))
    scale = HEAD_DIM ** -0.5 if softmax_scale is None else float(softmax_scale)
    out = torch.empty(b, s_q, h_q, HEAD_DIM_V, dtype=torch.bfloat16, device=q.device)
    lse = torch.empty(b, h_q, s_q, dtype=torch.float32, device=q.device)
    wsb = capi.mla_workspace_bytes(b, s_q, h_q, ns)
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=q.device)
    stream = torch.cuda.current_stream(q.device).cuda_stream
    rc = capi.mla_launch(q.data_ptr(), k_cache.data_ptr(), block_table.data_ptr(),
                         cache_seqlens.data_ptr(), out.data_ptr(), lse.data_ptr(), b, s_q, h_q, bs,
                         max_blocks, scale, int(bool(causal)), ns, ws.data_ptr(), wsb, stream)
    if rc != 0:
        raise RuntimeError(f"mla_decode_launch failed with HIP error {rc}")
    return out, lse
