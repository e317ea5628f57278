"""Page-table format conversion for library decode kernels.

The kernels here take a dense ``block_table [B, max_blocks]`` plus
``seq_lens [B]``. Paged-attention libraries usually take the compressed
(CSR) form instead: ``kv_indptr [B+1]``, ``kv_indices [sum_b n_b]`` and
``kv_last_page_len [B]`` with ``n_b = ceil(S_b / page_size)``. This module
converts between the two; the forward direction is the reference's
``block_table_to_paged`` (bench/baselines/flashinfer_adapter.py:33-51), with
its known-answer vector at tests/test_flashinfer_baseline.py:20-31.
"""

import torch


def pages_per_request(seq_lens, page_size):
    """n_b = ceil(S_b / page_size) as int32 (0 for S_b == 0)."""
    if page_size <= 0:
        raise ValueError(f"page_size must be positive, got {page_size}")
    return torch.div(seq_lens.to(torch.int64) + page_size - 1, page_size,
                     rounding_mode="floor").to(torch.int32)


def block_table_to_paged(block_table, seq_lens, page_size):
    """Dense table -> (kv_indptr [B+1], kv_indices [total], kv_last_page_len [B]).

    All three are int32 on block_table's device. kv_indices lists request b's
    first n_b block ids in logical order, requests in batch order; entries of
    block_table past n_b (padding, typically -1) are never read.
    kv_last_page_len[b] = S_b - (n_b - 1) * page_size, in [1, page_size] for
    S_b >= 1.
    """
    if block_table.dim() != 2 or seq_lens.dim() != 1 or block_table.shape[0] != seq_lens.shape[0]:
        raise ValueError("block_table must be [B, max_blocks] and seq_lens [B]")
    B, max_blocks = block_table.shape
    device = block_table.device
    seq_lens = seq_lens.to(device)
    n = pages_per_request(seq_lens, page_size)
    if B and int(n.max()) > max_blocks:
        raise ValueError("seq_lens needs more blocks than block_table holds")
    indptr = torch.zeros(B + 1, dtype=torch.int32, device=device)
    indptr[1:] = torch.cumsum(n, 0, dtype=torch.int32)
    keep = torch.arange(max_blocks, device=device)[None, :] < n[:, None]
    indices = block_table[keep].to(torch.int32)
    last_page_len = (seq_lens.to(torch.int32) - (n - 1) * page_size).to(torch.int32)
    return indptr, indices, last_page_len


def paged_to_block_table(indptr, indices, max_blocks=None, pad=-1):
    """Inverse of block_table_to_paged's first two outputs: CSR -> dense
    [B, max_blocks] int32 table, rows padded with `pad`."""
    B = indptr.numel() - 1
    n = (indptr[1:] - indptr[:-1]).to(torch.int64)
    width = int(n.max()) if B else 0
    if max_blocks is None:
        max_blocks = max(width, 1)
    if width > max_blocks:
        raise ValueError(f"a request holds {width} pages > max_blocks={max_blocks}")
    table = torch.full((B, max_blocks), pad, dtype=torch.int32, device=indices.device)
    keep = torch.arange(max_blocks, device=indices.device)[None, :] < n.to(indices.device)[:, None]
    table[keep] = indices.to(torch.int32)
    return table
