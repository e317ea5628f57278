/*
 * mla_decode_oracle.c -- CPU restatement of MLA absorbed-path paged decode.
 *
 * TEST INFRASTRUCTURE ONLY. Loaded by tests/ (checked against
 * oracle/mla_reference.py, which the closed forms, brute force and an
 * independent torch computation pin) and by bench.py's cpu_baseline leg for
 * the MLA configs (the timed CPU path). Nothing in the product links or
 * calls it.
 *
 * oracle_mla_decode follows oracle/mla_reference.py:mla_decode_ref, the
 * published decode semantics of FlashMLA (the reference's pinned K2 baseline,
 * docs/g0/flashmla_sha.txt; the reference's own kernels/mla_decode/ is
 * empty): per (b, query token i, head h), scores s_t = scale * <q, C_t> over
 * the request's first lim tokens (lim = S, or S - (s_q - 1 - i) when causal),
 * out = sum_t softmax(s)_t C_t[:dv], lse = log sum_t exp(s_t), in double
 * precision; a row with no key gets out = 0 and lse = -inf. C_t is the latent
 * row kv_cache[block_table[b, t / bs], t % bs, 0, :]. Rows are spread over
 * `nthreads` OpenMP threads (0: the runtime's default).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define MLA_D 576

static inline double bf16d(uint16_t u) {
  union {
    uint32_t u;
    float f;
  } x;
  x.u = (uint32_t)u << 16;
  return (double)x.f;
}

int oracle_mla_decode(const uint16_t* q, const uint16_t* kv_cache, const int32_t* block_table,
                      const int32_t* seq_lens, float* out, float* lse, int B, int s_q, int h_q,
                      int block_size, int max_blocks, int dv, float scale, int causal,
                      int nthreads) {
  if (B < 0 || s_q < 1 || h_q < 1 || block_size < 1 || max_blocks < 1 || dv < 1 || dv > MLA_D)
    return 1;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#endif
  const int64_t rows = (int64_t)B * s_q * h_q;
  int bad = 0;
#pragma omp parallel for schedule(dynamic, 4) reduction(| : bad)
  for (int64_t idx = 0; idx < rows; ++idx) {
    const int b = (int)(idx / ((int64_t)s_q * h_q));
    const int rem = (int)(idx - (int64_t)b * s_q * h_q);
    const int qi = rem / h_q, h = rem % h_q;
    const uint16_t* qv = q + idx * MLA_D;  /* [B, s_q, h_q, 576] */
    float* o = out + idx * dv;
    float* l_out = lse + ((int64_t)b * h_q + h) * s_q + qi;
    int S = seq_lens[b] > 0 ? seq_lens[b] : 0;
    if (S > block_size * max_blocks) S = block_size * max_blocks;
    const int lim = causal ? S - (s_q - 1 - qi) : S;
    for (int d = 0; d < dv; ++d) o[d] = 0.f;
    if (lim <= 0) {
      *l_out = -INFINITY;
      continue;
    }
    double* s = (double*)malloc(sizeof(double) * (size_t)lim);
    double* acc = (double*)calloc((size_t)dv, sizeof(double));
    if (!s || !acc) {
      free(s);
      free(acc);
      bad |= 1;
      continue;
    }
    double qd[MLA_D];
    for (int d = 0; d < MLA_D; ++d) qd[d] = bf16d(qv[d]);
    double m = -INFINITY;
    for (int t = 0; t < lim; ++t) {
      const int lb = t / block_size, slot = t % block_size;
      const uint16_t* c = kv_cache + ((int64_t)block_table[(int64_t)b * max_blocks + lb] *
                                          block_size + slot) * MLA_D;
      double dot = 0.0;
      for (int d = 0; d < MLA_D; ++d) dot += qd[d] * bf16d(c[d]);
      s[t] = dot * (double)scale;
      if (s[t] > m) m = s[t];
    }
    double l = 0.0;
    for (int t = 0; t < lim; ++t) {
      const double p = exp(s[t] - m);
      l += p;
      const int lb = t / block_size, slot = t % block_size;
      const uint16_t* c = kv_cache + ((int64_t)block_table[(int64_t)b * max_blocks + lb] *
                                          block_size + slot) * MLA_D;
      for (int d = 0; d < dv; ++d) acc[d] += p * bf16d(c[d]);
    }
    for (int d = 0; d < dv; ++d) o[d] = (float)(acc[d] / l);
    *l_out = (float)(m + log(l));
    free(s);
    free(acc);
  }
  return bad ? 2 : 0;
}
