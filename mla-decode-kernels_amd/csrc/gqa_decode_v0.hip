// v0: correctness-first decode kernel for gfx950.
//
// One wave64 per (b, q-head); lane i owns head dims {2i, 2i+1}. Tokens are
// visited one at a time with the fp32 online-softmax recurrence of the
// reference's v0 (kernels/gqa_decode/v0_naive.cu:6-25): the dot product is a
// full-wave reduction (4 DPP row steps + 2 cross-row shuffles, no LDS and no
// barriers), exp is the accurate expf, and the result is acc / l rounded to
// bf16. Its only purpose is to be obviously right; v1/v2 are the fast paths.
#include "gqa_device.hpp"
#include "gqa_launch.hpp"
#include "gqa_decode.h"

namespace gqa {

struct V0Args {
  const uint16_t* q;
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  const int* block_table;
  const int* seq_lens;
  uint16_t* out;
  int Hq, Hkv, block_size, max_blocks;
  float scale;
};

__global__ __launch_bounds__(64) void gqa_decode_v0_kernel(const V0Args a) {
  const int h = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  const int hkv = h / (a.Hq / a.Hkv);  // consecutive grouping (HF repeat_kv)
  const int S = a.seq_lens[b];

  const uint32_t qw = *reinterpret_cast<const uint32_t*>(
      a.q + ((size_t)b * a.Hq + h) * kHeadDim + 2 * lane);
  const float q0 = bf16_lo(qw), q1 = bf16_hi(qw);
  const uint32_t* k32 = reinterpret_cast<const uint32_t*>(a.k_cache);
  const uint32_t* v32 = reinterpret_cast<const uint32_t*>(a.v_cache);
  const int* bt = a.block_table + (size_t)b * a.max_blocks;

  float m = kNegInf, l = 0.f, acc0 = 0.f, acc1 = 0.f;
  for (int t = 0; t < S; ++t) {
    const int lb = t / a.block_size;
    const int slot = t - lb * a.block_size;
    const int64_t row = ((int64_t)bt[lb] * a.block_size + slot) * a.Hkv + hkv;
    const size_t w = (size_t)row * (kHeadDim / 2) + lane;
    const uint32_t kw = k32[w];
    const float sc = wave_sum(fmaf(q1, bf16_hi(kw), q0 * bf16_lo(kw))) * a.scale;
    const float m_new = fmaxf(m, sc);
    const float alpha = expf(m - m_new);
    const float p = expf(sc - m_new);
    const uint32_t vw = v32[w];
    l = fmaf(l, alpha, p);
    acc0 = fmaf(acc0, alpha, p * bf16_lo(vw));
    acc1 = fmaf(acc1, alpha, p * bf16_hi(vw));
    m = m_new;
  }
  const uint32_t lo = f32_to_bf16_bits(finalize(acc0, l));
  const uint32_t hi = f32_to_bf16_bits(finalize(acc1, l));
  reinterpret_cast<uint32_t*>(a.out + ((size_t)b * a.Hq + h) * kHeadDim)[lane] = lo | (hi << 16);
}

}  // namespace gqa

extern "C" int gqa_decode_v0_launch(const uint16_t* q, const uint16_t* k_cache,
                                    const uint16_t* v_cache, const int* block_table,
                                    const int* seq_lens, uint16_t* out, int B, int Hq, int Hkv,
                                    int block_size, int max_blocks, float scale,
                                    hipStream_t stream) {
  hipError_t err = gqa::check_common(q, k_cache, v_cache, block_table, seq_lens, out, B, Hq, Hkv,
                                     block_size, max_blocks);
  if (err != hipSuccess) return err;
  if (B == 0) return hipSuccess;
  const gqa::V0Args args{q, k_cache, v_cache, block_table, seq_lens, out,
                         Hq, Hkv, block_size, max_blocks, scale};
  hipLaunchKernelGGL(gqa::gqa_decode_v0_kernel, dim3(Hq, B), dim3(64), 0, stream, args);
  return hipGetLastError();
}
