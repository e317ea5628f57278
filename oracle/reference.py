"""CPU oracle for paged GQA decode attention -- test infrastructure only.

This module is the checker the tests, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` compare the HIP kernels against. It is
never on the product path: the kernels are reached only through
``include/gqa_decode.h`` and fail loudly when the library is missing.

It restates, in numpy, the reference's fp32 oracle and the split-KV state
semantics (paths relative to the reference checkout):

  gather_kv        python/reference.py:7-18
  attention_ref    python/reference.py:21-40
  partial_state    kernels/gqa_decode/v2_splitkv.cu:30-40,50-89 (one segment's
                   unnormalised (m, l, acc); empty segment -> (-inf, 0, 0))
  merge_states     kernels/gqa_decode/v2_splitkv.cu:92-108
  split_bounds     kernels/gqa_decode/v2_splitkv.cu:30-32
  kv_row_offset    kernels/gqa_decode/v0_naive.cu:16-17, docs/k1/notes_w1.md:53-72

bf16 tensors are carried as uint16 arrays of raw bf16 bits (numpy has no
bf16); ``bf16_to_f32`` widens them exactly.

How each function is pinned (tests/test_oracle.py):
  kv_row_offset / gather_kv  the notes_w1.md:59-68 worked example (element
                             37,248, byte 74,496), self-describing caches
                             whose values encode their own index, NaN in
                             every slot that must not be read.
  attention_ref              torch SDPA with repeat_interleave (the reference's
                             own check, tests/test_reference.py:13-23, < 1e-5);
                             float64 brute force on tiny inputs; closed forms
                             (S=1 -> V[0], identical keys -> mean V, one
                             dominant key -> its V row); the notes_w1.md:74-86
                             online-softmax trace; a head-map case that fails
                             for kv = h % Hkv.
  partial_state/merge_states the notes_w1.md:88-95 split-merge trace; merge of
                             any split equals attention_ref; empty segments.
  f32_to_bf16                torch's .to(torch.bfloat16) (round to nearest even).
"""

import math

import numpy as np

D = 128


def bf16_to_f32(bits):
    """Raw bf16 bits (uint16 array) -> float32, exactly."""
    bits = np.asarray(bits, dtype=np.uint16)
    return (bits.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x):
    """float32 -> raw bf16 bits, round to nearest even; NaN stays NaN."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    rounded[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return rounded


def kv_row_offset(block_table_row, t, block_size, Hkv, hkv):
    """Element offset of token t's (kv-head hkv) row in an NHD paged cache:
    ((p*bs + s)*Hkv + hkv)*D with p = block_table_row[t // bs], s = t % bs."""
    lb, s = divmod(int(t), int(block_size))
    p = int(block_table_row[lb])
    return ((p * int(block_size) + s) * int(Hkv) + int(hkv)) * D


def gather_kv(k_cache, v_cache, block_table, seq_len, b):
    """First seq_len tokens of request b from the paged caches, as float32
    arrays [seq_len, Hkv, D]. Only blocks block_table[b, :ceil(seq_len/bs)]
    and, in the last one, only its first seq_len - (n-1)*bs slots are read."""
    bs = k_cache.shape[1]
    n = (int(seq_len) + bs - 1) // bs
    blocks = np.asarray(block_table[b, :n], dtype=np.int64)
    Hkv = k_cache.shape[2]
    K = k_cache[blocks].reshape(n * bs, Hkv, D)[:seq_len]
    V = v_cache[blocks].reshape(n * bs, Hkv, D)[:seq_len]
    if K.dtype == np.uint16:
        K, V = bf16_to_f32(K), bf16_to_f32(V)
    return K.astype(np.float32, copy=False), V.astype(np.float32, copy=False)


def _softmax(scores):
    e = np.exp(scores - scores.max())
    return e / e.sum()


def attention_ref(q, k_cache, v_cache, block_table, seq_lens, scale, batches=None):
    """fp32 reference: out[b, h] = softmax(K[:, kv] @ q[b, h] * scale) @ V[:, kv]
    with kv = h // (Hq // Hkv). Returns float32 [B, Hq, D] (only the rows in
    `batches` are filled when that subset is given; the rest are NaN)."""
    q = np.asarray(q)
    B, Hq, _ = q.shape
    Hkv = k_cache.shape[2]
    G = Hq // Hkv
    qf = bf16_to_f32(q) if q.dtype == np.uint16 else q.astype(np.float32)
    out = np.full((B, Hq, D), np.nan, dtype=np.float32)
    for b in range(B) if batches is None else batches:
        S = int(seq_lens[b])
        K, V = gather_kv(k_cache, v_cache, block_table, S, b)
        for h in range(Hq):
            kv = h // G
            scores = (K[:, kv, :] @ qf[b, h]) * np.float32(scale)
            w = _softmax(scores.astype(np.float32))
            out[b, h] = w @ V[:, kv, :]
    return out


def partial_state(q_vec, K, V, scale):
    """Unnormalised online-softmax state of one segment, natural-log units:
    m = max_t s_t, l = sum_t exp(s_t - m), acc = sum_t exp(s_t - m) V_t with
    s_t = scale * <q, K_t>. An empty segment gives (-inf, 0, zeros)."""
    K = np.asarray(K, dtype=np.float64)
    V = np.asarray(V, dtype=np.float64)
    if K.shape[0] == 0:
        return -math.inf, 0.0, np.zeros(V.shape[1] if V.ndim == 2 else D)
    s = (K @ np.asarray(q_vec, dtype=np.float64)) * float(scale)
    m = float(s.max())
    e = np.exp(s - m)
    return m, float(e.sum()), e @ V


def merge_states(ms, ls, accs):
    """Log-sum-exp merge of segment states in the given order:
    M = max m_i, L = sum l_i e^(m_i - M), out = sum acc_i e^(m_i - M) / L.
    Segments with m_i = -inf contribute factor 0."""
    ms = np.asarray(ms, dtype=np.float64)
    M = ms.max()
    f = np.where(ms == -np.inf, 0.0, np.exp(ms - M))
    L = float((np.asarray(ls, dtype=np.float64) * f).sum())
    acc = (np.asarray(accs, dtype=np.float64) * f[:, None]).sum(axis=0)
    return acc / L, M, L


def split_bounds(S, num_splits):
    """The reference's segment rule: chunk = ceil(S / ns), segment i covers
    [i*chunk, min(S, (i+1)*chunk)); segments starting at or past S are empty."""
    chunk = (int(S) + num_splits - 1) // num_splits
    return [(min(i * chunk, S), min(S, (i + 1) * chunk)) for i in range(num_splits)]
