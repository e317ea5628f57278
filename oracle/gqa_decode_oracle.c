/*
 * gqa_decode_oracle.c -- CPU restatement of the reference's fp32 oracle.
 *
 * TEST INFRASTRUCTURE ONLY. Loaded by tests/ (as a second, independent
 * restatement checked against oracle/reference.py and the known-answer
 * vectors) and by bench.py's cpu_baseline leg (the timed CPU path). Nothing
 * in the product links or calls it.
 *
 * oracle_attention_ref restates python/reference.py:21-40 (with the gather of
 * :7-18 done by index arithmetic, kernels/gqa_decode/v0_naive.cu:16-17): per
 * (b, q-head), scores s_t = scale * <q, K_t> over the request's first S
 * tokens, w = softmax(s) (exp(s - max) / sum), out = sum_t w_t V_t, all in
 * fp32 with libm expf; kv-head = h / (Hq / Hkv). The (b, q-head) pairs are
 * independent and are spread over `nthreads` OpenMP threads.
 *
 * oracle_partial_state / oracle_merge_states restate the split-KV state and
 * merge of kernels/gqa_decode/v2_splitkv.cu:30-40,50-89 and :92-108 in double
 * precision.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define ORACLE_D 128

static inline float bf16f(uint16_t u) {
  union {
    uint32_t u;
    float f;
  } x;
  x.u = (uint32_t)u << 16;
  return x.f;
}

/* Element offset of token t's kv-head row: ((p*bs + s)*Hkv + hkv)*D. */
int64_t oracle_kv_offset(const int32_t* bt_row, int t, int block_size, int Hkv, int hkv) {
  const int lb = t / block_size, s = t % block_size;
  return (((int64_t)bt_row[lb] * block_size + s) * Hkv + hkv) * ORACLE_D;
}

static void one_head(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                     const int32_t* bt_row, int S, int block_size, int Hkv, int hkv, float scale,
                     float* scores, float* out) {
  float qf[ORACLE_D];
  for (int d = 0; d < ORACLE_D; ++d) qf[d] = bf16f(q[d]);
  float mx = -INFINITY;
  for (int t = 0; t < S; ++t) {
    const uint16_t* k = k_cache + oracle_kv_offset(bt_row, t, block_size, Hkv, hkv);
    float acc = 0.f;
#pragma omp simd reduction(+ : acc)
    for (int d = 0; d < ORACLE_D; ++d) acc += qf[d] * bf16f(k[d]);
    scores[t] = acc * scale;
    if (scores[t] > mx) mx = scores[t];
  }
  float sum = 0.f;
  for (int t = 0; t < S; ++t) {
    scores[t] = expf(scores[t] - mx);
    sum += scores[t];
  }
  float o[ORACLE_D];
  memset(o, 0, sizeof(o));
  for (int t = 0; t < S; ++t) {
    const float w = scores[t] / sum;
    const uint16_t* v = v_cache + oracle_kv_offset(bt_row, t, block_size, Hkv, hkv);
#pragma omp simd
    for (int d = 0; d < ORACLE_D; ++d) o[d] += w * bf16f(v[d]);
  }
  memcpy(out, o, sizeof(o));
}

/* out [B, Hq, 128] fp32. Returns 0, or -1 on bad arguments / allocation. */
int oracle_attention_ref(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                         const int32_t* block_table, const int32_t* seq_lens, float* out, int B,
                         int Hq, int Hkv, int block_size, int max_blocks, float scale,
                         int nthreads) {
  if (B < 0 || Hq < 1 || Hkv < 1 || Hq % Hkv != 0 || block_size < 1 || max_blocks < 1) return -1;
  int smax = 0;
  for (int b = 0; b < B; ++b) {
    if (seq_lens[b] < 0 || seq_lens[b] > max_blocks * block_size) return -1;
    if (seq_lens[b] > smax) smax = seq_lens[b];
  }
  const int G = Hq / Hkv;
  const int64_t pairs = (int64_t)B * Hq;
  int failed = 0;
#ifdef _OPENMP
  if (nthreads < 1) nthreads = omp_get_max_threads();
#pragma omp parallel num_threads(nthreads) reduction(| : failed)
#endif
  {
    float* scores = (float*)malloc(sizeof(float) * (size_t)(smax > 0 ? smax : 1));
    if (!scores) {
      failed = 1;
    } else {
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
      for (int64_t i = 0; i < pairs; ++i) {
        const int b = (int)(i / Hq), h = (int)(i % Hq);
        one_head(q + i * ORACLE_D, k_cache, v_cache, block_table + (int64_t)b * max_blocks,
                 seq_lens[b], block_size, Hkv, h / G, scale, scores, out + i * ORACLE_D);
      }
      free(scores);
    }
  }
  return failed ? -1 : 0;
}

/* Unnormalised state of tokens [start, end) for one (q vector, kv-head):
 * m = max s_t, l = sum e^(s_t - m), acc = sum e^(s_t - m) V_t (natural-log
 * units, double accumulation). Empty range -> (-inf, 0, 0). */
void oracle_partial_state(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                          const int32_t* bt_row, int block_size, int Hkv, int hkv, int start,
                          int end, float scale, double* m, double* l, double* acc) {
  *m = -INFINITY;
  *l = 0.0;
  for (int d = 0; d < ORACLE_D; ++d) acc[d] = 0.0;
  for (int t = start; t < end; ++t) {
    const uint16_t* k = k_cache + oracle_kv_offset(bt_row, t, block_size, Hkv, hkv);
    double s = 0.0;
    for (int d = 0; d < ORACLE_D; ++d) s += (double)bf16f(q[d]) * bf16f(k[d]);
    s *= scale;
    if (s > *m) *m = s;
  }
  for (int t = start; t < end; ++t) {
    const int64_t off = oracle_kv_offset(bt_row, t, block_size, Hkv, hkv);
    double s = 0.0;
    for (int d = 0; d < ORACLE_D; ++d) s += (double)bf16f(q[d]) * bf16f(k_cache[off + d]);
    const double w = exp(s * scale - *m);
    *l += w;
    for (int d = 0; d < ORACLE_D; ++d) acc[d] += w * bf16f(v_cache[off + d]);
  }
}

/* Merge ns states in order: M = max m_i, factor_i = e^(m_i - M) (0 for
 * m_i = -inf), out = sum factor_i acc_i / sum factor_i l_i. `width` is the
 * acc vector length. */
void oracle_merge_states(int ns, const double* m, const double* l, const double* acc, int width,
                         double* out) {
  double M = -INFINITY, L = 0.0;
  for (int i = 0; i < ns; ++i)
    if (m[i] > M) M = m[i];
  for (int d = 0; d < width; ++d) out[d] = 0.0;
  for (int i = 0; i < ns; ++i) {
    const double f = m[i] == -INFINITY ? 0.0 : exp(m[i] - M);
    L += l[i] * f;
    for (int d = 0; d < width; ++d) out[d] += acc[(int64_t)i * width + d] * f;
  }
  for (int d = 0; d < width; ++d) out[d] /= L;
}
