"""CPU oracle for MLA absorbed-path paged decode -- test infrastructure only.

The checker that the MLA tests, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` compare the HIP kernel against. It is
never on the product path (the kernel is reached only through
``include/mla_decode.h``).

The reference has no MLA implementation: ``kernels/mla_decode/`` is an empty
placeholder and ``README.md:405-408`` (paths relative to the reference
checkout) names the item -- "MLA absorbed-path paged decode: latent cache
[num_blocks, 64, 576]" -- with FlashMLA at 15f13e5 (``docs/g0/flashmla_sha.txt``)
as its baseline. FlashMLA is a third-party dependency absent from the
reference; this module restates its published decode semantics
(``flash_mla_with_kvcache``):

  out[b, i, h]  = softmax_t(scale * <q[b, i, h], C_b[t]>) . C_b[t, :dv]
  lse[b, h, i]  = logsumexp_t(scale * <q[b, i, h], C_b[t]>)   (natural log)
  C_b[t]        = kv_cache[block_table[b, t // bs], t % bs, 0]   (one latent head)

for t < seq_lens[b], or with causal=True for t < seq_lens[b] - (s_q - 1 - i).
A row with no key gets out = 0 and lse = -inf. Arithmetic is float64 on the
bf16 inputs widened exactly.

How it is pinned (tests/test_mla_oracle.py): closed forms (one token -> its
value row; identical keys -> the mean of the values; a single dominant key),
float64 brute force over explicit loops on tiny inputs, an independent torch
float32 computation through torch.nn.functional.scaled_dot_product_attention
with an explicit mask, the paged gather against a contiguous cache, and the
causal mask against per-query truncation of the sequence.
"""

import numpy as np

from oracle.reference import bf16_to_f32

D = 576
DV = 512


def gather_latent(kv_cache, block_table_row, seq_len):
    """Rows t < seq_len of one request's latent cache: [seq_len, 576] float32
    (bf16 bits widened). kv_cache is [num_blocks, bs, 1, 576] uint16."""
    bs = kv_cache.shape[1]
    n = (int(seq_len) + bs - 1) // bs
    blocks = np.asarray(block_table_row[:n], dtype=np.int64)
    rows = kv_cache[blocks, :, 0, :].reshape(n * bs, D)[:int(seq_len)]
    return bf16_to_f32(rows)


def mla_decode_ref(q, kv_cache, block_table, seq_lens, scale, causal=False, dv=DV, batches=None):
    """Reference MLA decode. q: [B, s_q, h_q, 576] uint16 (bf16 bits);
    kv_cache: [num_blocks, bs, 1, 576] uint16; block_table [B, max_blocks]
    int32; seq_lens [B]. Returns (out [nb, s_q, h_q, dv] float32,
    lse [nb, h_q, s_q] float32) for the requests in `batches` (all by
    default)."""
    B, s_q, h_q, _ = q.shape
    batches = list(range(B)) if batches is None else list(batches)
    out = np.zeros((len(batches), s_q, h_q, dv), np.float64)
    lse = np.full((len(batches), h_q, s_q), -np.inf, np.float64)
    for i, b in enumerate(batches):
        S = max(int(seq_lens[b]), 0)
        if S == 0:
            continue
        C = gather_latent(kv_cache, block_table[b], S).astype(np.float64)
        Q = bf16_to_f32(q[b]).astype(np.float64)          # [s_q, h_q, 576]
        scores = np.einsum("ihd,td->iht", Q, C) * scale    # [s_q, h_q, S]
        for qi in range(s_q):
            lim = S - (s_q - 1 - qi) if causal else S
            if lim <= 0:
                continue
            s = scores[qi, :, :lim]
            m = s.max(axis=1, keepdims=True)
            p = np.exp(s - m)
            l = p.sum(axis=1, keepdims=True)
            out[i, qi] = (p / l) @ C[:lim, :dv]
            lse[i, :, qi] = (m + np.log(l))[:, 0]
    return out.astype(np.float32), lse.astype(np.float32)
