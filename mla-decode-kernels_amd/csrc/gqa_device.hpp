// Device helpers shared by the gfx950 GQA decode kernels: bf16 unpacking,
// 16-lane DPP reductions, base-2 exponential, division by a runtime constant,
// and the output normalisation every kernel ends with.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gqa {

constexpr int kHeadDim = 128;
constexpr float kNegInf = -__builtin_inff();
// log2(e) and ln(2): the kernels evaluate exp(x) as 2^(x*log2(e)) on the
// hardware base-2 exponential (v_exp_f32), the usual flash-decoding method.
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// The two bf16 values packed in one 32-bit word, widened exactly to fp32.
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16, round to nearest even (the rounding of __float2bfloat16 and of
// torch's .to(torch.bfloat16)); NaN stays NaN.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// 16-byte load of K/V cache data with the non-temporal hint
// (global_load_dwordx4 ... nt). A decode step reads every cache row exactly
// once, so the rows are a pure stream; measured on MI355X with the kernels'
// own access pattern (256-byte head rows at a 2 KiB slot stride, 16-byte
// loads, one wave per SIMD, 1 GiB), the hint raises the read rate from
// 5.97 to 7.04 TB/s.
__device__ __forceinline__ uint4 load_kv(const uint16_t* p) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// The same streaming load through a raw buffer resource: a uniform base in
// SGPRs plus a 32-bit per-lane byte offset, so no 64-bit address arithmetic
// per load. kv_rsrc(base) covers [base, base + 4 GiB) (stride 0; the last
// descriptor word is the gfx9-family raw-buffer format); cache-policy value 2
// sets nt.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t kv_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, -1, 0x00020000);
}
__device__ __forceinline__ uint4 load_kv(__amdgpu_buffer_rsrc_t rsrc, uint32_t byte_off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, byte_off, 0, 2));
}

// acc += <a, b> over two packed bf16 pairs (v_dot2c_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), acc, false);
}

template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kCtrl, 0xF, 0xF, true));
}

// Sum over the 16 lanes of each DPP row; every lane of the row receives the
// bitwise-identical total (each step adds a value to its mirror image, and fp
// addition is commutative), so all lanes then take the same softmax path.
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_f32<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp_f32<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp_f32<0x141>(x);  // row_half_mirror
  x += dpp_f32<0x140>(x);  // row_mirror
  return x;
}

// Cross-row exchanges on gfx950's lane-swap instructions. v_permlane16_swap_b32
// swaps the odd 16-lane rows of its first operand with the even rows of its
// second, v_permlane32_swap_b32 the upper 32 lanes of its first operand with
// the lower 32 lanes of its second (pinned on the GPU by issue_probe's lane
// probe). With x as both operands, lane l holds x[l] in one result and
// x[l ^ 16] (x[l ^ 32]) in the other, so a commutative op of the two results
// gives op(x[l], x[l ^ 16]) -- the bits of x op __shfl_xor(x, 16) -- in two
// VALU instructions, where the shuffle is an LDS permute and a wait on it.
__device__ __forceinline__ void xor16_pair(float x, float& a, float& b) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  a = __uint_as_float(p[0]);
  b = __uint_as_float(p[1]);
}
__device__ __forceinline__ void xor32_pair(float x, float& a, float& b) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  a = __uint_as_float(p[0]);
  b = __uint_as_float(p[1]);
}
// x[l] + x[l ^ 16], x[l] + x[l ^ 32], and the maxima, in every lane l.
__device__ __forceinline__ float xor16_sum(float x) {
  float a, b;
  xor16_pair(x, a, b);
  return a + b;
}
__device__ __forceinline__ float xor32_sum(float x) {
  float a, b;
  xor32_pair(x, a, b);
  return a + b;
}
__device__ __forceinline__ float xor16_max(float x) {
  float a, b;
  xor16_pair(x, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float xor32_max(float x) {
  float a, b;
  xor32_pair(x, a, b);
  return fmaxf(a, b);
}

// Sum over all 64 lanes, identical in every lane.
__device__ __forceinline__ float wave_sum(float x) { return xor32_sum(xor16_sum(row16_sum(x))); }

// Max over all 64 lanes, identical in every lane (max is exact, so the order
// of the steps does not matter).
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, dpp_f32<0xB1>(x));
  x = fmaxf(x, dpp_f32<0x4E>(x));
  x = fmaxf(x, dpp_f32<0x141>(x));
  x = fmaxf(x, dpp_f32<0x140>(x));
  return xor32_max(xor16_max(x));
}

// Hardware 2^x (v_exp_f32): 2^-inf = 0, 2^0 = 1.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Quotient n / d for 0 <= n < 2^31 and a divisor fixed at launch time, by the
// round-up multiply-shift method (Granlund & Montgomery, PLDI 1994, sec. 4):
// with l = ceil(log2 d) and mul = floor(2^32 (2^l - d) / d) + 1,
// n / d == (umulhi(n, mul) + n) >> l.
struct FastDiv {
  uint32_t d, mul, shift;
};

inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  const uint64_t mul = ((1ull << 32) * ((1ull << l) - d)) / d + 1;
  return FastDiv{d, (uint32_t)mul, l};
}

__device__ __forceinline__ uint32_t fastdiv(uint32_t n, const FastDiv& f) {
  return (__umulhi(n, f.mul) + n) >> f.shift;
}

// The single normalisation step every kernel finishes with (out = acc / l).
// The single-pass and split-KV paths both call it, so a one-split merge (whose
// factor is exactly 1) reproduces the single-pass output bit for bit.
__device__ __forceinline__ float finalize(float acc, float l) { return acc / l; }

}  // namespace gqa
