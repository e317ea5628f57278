// The matrix-core scan of one (request, kv-head) segment by one wave: tile
// loads, QK^T and PV on MFMA, online softmax on the MFMA C layout. Shared by
// the split-rule kernel (gqa_decode_mfma.hip) and the token-balanced kernel
// (gqa_decode_balanced.hip); everything here is force-inlined into them.
//
// A tile is 16 (or 32) tokens of one kv-head:
//
//   QK^T   S^T[16 tok x 16 heads] = K[tok x 128] . Q^T[128 x 16 heads], four
//          v_mfma_f32_16x16x32_bf16 (K-steps of 32 dims) per 16 tokens.
//          A = K rows straight from HBM (lane l: token l%16, dims
//          32kk + 8(l/16) .. +8, one 16-byte load), B = Q^T held in registers
//          (lane l: head l%16). Up to 16 q-heads share one MFMA, so a group of
//          up to 16 reads its K/V once; heads past the group carry q = 0 and
//          are never written.
//   softmax on the C layout: lane l owns head l%16 and tokens 4(l/16)+e,
//          e < 4 (+16 per further token group); one max / rescale per tile.
//   PV     O[16 heads x 128 dims] += P[heads x tok] . V[tok x dims], eight
//          MFMAs of 16 dims: v_mfma_f32_16x16x16_bf16 for 16-token tiles
//          (P is already the A operand: head l%16, tokens 4(l/16)..+3), or
//          16x16x32 for 32-token tiles under the token permutation
//          k-slot 8g+e -> token 4g+e, 8g+4+e -> token 16+4g+e. P enters as
//          two bf16 parts, P = P_hi + P_lo (P_hi = bf16(P); P_lo = bf16 of the
//          remainder P - P_hi, which is exact in fp32), each multiplied by V
//          on its own MFMA: the effective weight P_hi + P_lo is within 2^-18
//          relative of the fp32 one (a single bf16 part: 2^-9), which keeps the
//          PV product as accurate as the reference's fp32 p * V
//          (v2_splitkv.cu:60-63) to within fp32 summation noise. The fp32
//          sum l accumulates the same effective weights, so the weights stay
//          normalised. The V tile goes through
//          LDS: written row-major with a 16-byte-chunk XOR swizzle and read
//          back with ds_read_b64_tr_b16, whose 16-lane transpose hands lane l
//          the 4 consecutive tokens of dim l%16 that the B operand needs
//          (lane x supplies row T + x/4, column 4(x%4)).
//
// State stays fp32: m per head (base-2 units), l and O accumulated in fp32.
#pragma once

#include "gqa_device.hpp"
#include "gqa_scan.hpp"

namespace gqa {

constexpr int kMHeads = 16;  // q-heads per MFMA column block
// Tokens per wave per tile (16 or 32). Measured: 16-token tiles (one tile in
// flight per wave, as in the VALU scan) beat 32-token ones by 1-12% in both
// launch layouts.
#ifndef GQA_MFMA_TILE
#define GQA_MFMA_TILE 16
#endif
constexpr int kMTile = GQA_MFMA_TILE;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4_t;

template <int NG>
struct MTileRegs {
  uint4 k[NG][4];  // [16-token group][32-dim step]: A operands of the QK MFMAs
  uint4 v[4 * NG]; // V: load i holds token 4i + lane/16, dims 8*(lane%16) .. +8
};

// One wave's scan state. Lane l = (j = l%16, g = l/16): m and lsum belong to
// head j (lsum over this lane's token slots only), o[nb][e] is
// O[head 4g + e][dim 16nb + j].
struct MfmaState {
  float m, lsum;
  f32x4_t o[8];
};

__device__ __forceinline__ void mfma_init(MfmaState& st) {
  st.m = kNegInf;
  st.lsum = 0.f;
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) st.o[nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
}

__device__ __forceinline__ bf16x8_t as_bf16x8(const uint4& u) {
  return __builtin_bit_cast(bf16x8_t, u);
}

// Byte offset of 16-byte chunk c (dims 8c .. 8c+8) of tile row r in a wave's
// V buffer. The XOR keeps the 8 rows a half-wave transpose-reads at one
// column on 8 different 16-byte bank groups.
__device__ __forceinline__ uint32_t vlds_offset(int r, int c) {
  return (uint32_t)r * 256u + (uint32_t)((c ^ ((r & 7) << 1)) << 4);
}

// Hand LDS data from some lanes of a wave to others: wait for the wave's LDS
// operations (s_waitcnt lgkmcnt(0); vmcnt / expcnt untouched, gfx9 encoding)
// and keep the compiler from moving memory accesses across the point.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// B operands of the QK MFMAs for q-heads h0 .. h0 + nh - 1 of request b:
// Q^T, lane (j, g) holds head h0 + j, dims 32kk + 8g .. +8 (zero past nh).
__device__ __forceinline__ void mfma_load_q(const ScanArgs& a, int b, int h0, int nh, int j, int g,
                                            uint4 (&qf)[4]) {
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    qf[kk] = make_uint4(0, 0, 0, 0);
    if (j < nh)
      qf[kk] = *reinterpret_cast<const uint4*>(a.q + ((size_t)b * a.Hq + h0 + j) * kHeadDim +
                                               32 * kk + 8 * g);
  }
}

// Scan tokens [seg_start, seg_end) of kv-head hkv of the request whose block
// table row is bt: the wave takes tiles first, first + stride, ... and folds
// them into st, staging V through its own T * 256-byte LDS buffer vbuf. The
// next tile's loads are issued before the current tile is consumed.
template <int T, bool kBlockUniform>
__device__ __forceinline__ void mfma_scan_segment(const ScanArgs& a, const int* bt, int hkv,
                                                  const uint4 (&qf)[4], int seg_start, int seg_end,
                                                  int first, int stride, uint8_t* vbuf, int j,
                                                  int g, MfmaState& st) {
  constexpr int NG = T / 16;  // 16-token groups per tile
  const int ntiles = (seg_end - seg_start + T - 1) / T;
  const int my_tiles = ntiles > first ? (ntiles - first + stride - 1) / stride : 0;
  const uint32_t row_elems = (uint32_t)a.Hkv * kHeadDim;
  // The table is read-only for the launch. Reading it through the constant
  // address space makes the uniform block-id load scalar: as a vector load it
  // would share vmcnt with the tile loads, and waiting for it would drain every
  // load in flight (measured: 2-3% on 64Q/8KV, S=32768).
  const __attribute__((address_space(4))) int* btc =
      (const __attribute__((address_space(4))) int*)bt;
  const int bs = a.block_size;
  const size_t head_off = (size_t)hkv * kHeadDim;

  auto tile_start = [&](int k) { return seg_start + T * (first + stride * k); };

  // Element offset of token t's kv-head row (generic block sizes).
  auto row_of = [&](int t) -> size_t {
    const uint32_t lb = fastdiv((uint32_t)t, a.bs_div);
    const int slot = t - (int)lb * bs;
    return ((size_t)bt[lb] * bs + slot) * row_elems + head_off;
  };

  // Loads of tile k. Tokens at or past seg_end read a valid token of the tile
  // instead (their scores are masked), so nothing outside the request's live
  // slots is touched.
  auto issue = [&](int k, MTileRegs<NG>& t) {
    const int ts = tile_start(k);
    if constexpr (kBlockUniform) {
#pragma unroll
      for (int tg = 0; tg < NG; ++tg) {
        // 16 tokens from a 16-aligned start share one block.
        const int tb = ts + 16 * tg < seg_end ? ts + 16 * tg : ts;
        const uint32_t lb = fastdiv((uint32_t)tb, a.bs_div);
        const uint32_t slot0 = (uint32_t)(tb - (int)lb * bs);
        const size_t blk = (size_t)btc[lb] * ((size_t)bs * row_elems) + head_off;
        const uint32_t sk = ts + 16 * tg + j < seg_end ? slot0 + j : slot0;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
          t.k[tg][kk] = load_kv(a.k_cache + blk + sk * row_elems + 32 * kk + 8 * g);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t sv = ts + 16 * tg + 4 * i + g < seg_end ? slot0 + 4 * i + g : slot0;
          t.v[4 * tg + i] = load_kv(a.v_cache + blk + sv * row_elems + 8 * j);
        }
      }
    } else {
#pragma unroll
      for (int tg = 0; tg < NG; ++tg) {
        int tk = ts + 16 * tg + j;
        tk = tk < seg_end ? tk : ts;
        const size_t rk = row_of(tk);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
          t.k[tg][kk] = load_kv(a.k_cache + rk + 32 * kk + 8 * g);
      }
#pragma unroll
      for (int i = 0; i < 4 * NG; ++i) {
        int tv = ts + 4 * i + g;
        tv = tv < seg_end ? tv : ts;
        t.v[i] = load_kv(a.v_cache + row_of(tv) + 8 * j);
      }
    }
  };

  auto consume = [&](int k, const MTileRegs<NG>& t) {
    const int ts = tile_start(k);
    // Stage V (row-major, swizzled) for the transposed reads below.
#pragma unroll
    for (int i = 0; i < 4 * NG; ++i)
      *reinterpret_cast<uint4*>(vbuf + vlds_offset(4 * i + g, j)) = t.v[i];

    // QK^T: c[tg][e] = score of token 16tg + 4g + e for head j.
    f32x4_t c[NG];
#pragma unroll
    for (int tg = 0; tg < NG; ++tg) {
      c[tg] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        c[tg] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(t.k[tg][kk]), as_bf16x8(qf[kk]),
                                                        c[tg], 0, 0, 0);
    }
    float s[NG][4];
    float mx = kNegInf;
#pragma unroll
    for (int tg = 0; tg < NG; ++tg)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool valid = ts + 16 * tg + 4 * g + e < seg_end;
        s[tg][e] = valid ? c[tg][e] * a.scale_log2e : kNegInf;
        mx = fmaxf(mx, s[tg][e]);
      }
    mx = xor32_max(xor16_max(mx));
    const float mn = fmaxf(st.m, mx);
    const float ms = mn == kNegInf ? 0.f : mn;
    const float alpha = exp2_fast(st.m - ms);
    st.m = mn;

    // P as bf16 pairs P_hi + P_lo: per 16-token group, k-slots 4g..4g+3 =
    // tokens 4g..4g+3.
    uint32_t pw[2 * NG], pl[2 * NG];
    float psum = 0.f;
#pragma unroll
    for (int tg = 0; tg < NG; ++tg)
#pragma unroll
      for (int e = 0; e < 4; e += 2) {
        const f32x2_t pf = {exp2_fast(s[tg][e] - ms), exp2_fast(s[tg][e + 1] - ms)};
        const uint32_t w = __builtin_bit_cast(uint32_t, __builtin_convertvector(pf, bf16x2_t));
        const f32x2_t rem = {pf[0] - bf16_lo(w), pf[1] - bf16_hi(w)};
        const uint32_t wl = __builtin_bit_cast(uint32_t, __builtin_convertvector(rem, bf16x2_t));
        pw[2 * tg + e / 2] = w;
        pl[2 * tg + e / 2] = wl;
        psum += (bf16_lo(w) + bf16_lo(wl)) + (bf16_hi(w) + bf16_hi(wl));
      }
    st.lsum = fmaf(st.lsum, alpha, psum);

    // Rescale O rows (heads 4g + e) when any head's max moved.
    if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
      float ae[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) ae[e] = __shfl(alpha, 4 * g + e, 64);
#pragma unroll
      for (int nb = 0; nb < 8; ++nb)
#pragma unroll
        for (int e = 0; e < 4; ++e) st.o[nb][e] *= ae[e];
    }

    wave_lds_sync();
    // PV: B operand of dim block nb = V[tokens of k-slots][dim 16nb + j], read
    // transposed: lane x supplies row 4g + x/4 (+16 per token group).
    // The P_hi products of all 8 dim blocks come first, then the P_lo ones, so
    // no MFMA waits for the one before it.
    const int rr = 4 * g + (j >> 2);
    if constexpr (NG == 1) {
      // K = 16 tokens: A = P (lane: head j, tokens 4g..4g+3), B = V (dim j).
      bf16x4_t vb[8];
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) {
        const int cc = 2 * nb + ((j & 3) >> 1);
        vb[nb] = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (lds_bf16x4_t*)(vbuf + vlds_offset(rr, cc) + 8u * (j & 1)));
        st.o[nb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
            __builtin_bit_cast(bf16x4_t, make_uint2(pw[0], pw[1])), vb[nb], st.o[nb], 0, 0, 0);
      }
#pragma unroll
      for (int nb = 0; nb < 8; ++nb)
        st.o[nb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
            __builtin_bit_cast(bf16x4_t, make_uint2(pl[0], pl[1])), vb[nb], st.o[nb], 0, 0, 0);
    } else {
      // K = 32 tokens, k-slot 8g+e -> token 4g+e, 8g+4+e -> token 16+4g+e.
      bf16x8_t vb[8];
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) {
        const int cc = 2 * nb + ((j & 3) >> 1);
        const uint32_t half = 8u * (j & 1);
        const bf16x4_t v0 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (lds_bf16x4_t*)(vbuf + vlds_offset(rr, cc) + half));
        const bf16x4_t v1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (lds_bf16x4_t*)(vbuf + vlds_offset(rr + 16, cc) + half));
        vb[nb] = bf16x8_t{v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
        st.o[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            as_bf16x8(make_uint4(pw[0], pw[1], pw[2], pw[3])), vb[nb], st.o[nb], 0, 0, 0);
      }
#pragma unroll
      for (int nb = 0; nb < 8; ++nb)
        st.o[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            as_bf16x8(make_uint4(pl[0], pl[1], pl[2], pl[3])), vb[nb], st.o[nb], 0, 0, 0);
    }
    wave_lds_sync();
  };

  if (my_tiles > 0) {
    MTileRegs<NG> t0, t1;
    issue(0, t0);
    int k = 0;
    for (; k + 2 < my_tiles; k += 2) {
      issue(k + 1, t1);
      consume(k, t0);
      issue(k + 2, t0);
      consume(k + 1, t1);
    }
    if (k + 1 < my_tiles) {
      issue(k + 1, t1);
      consume(k, t0);
      consume(k + 1, t1);
    } else {
      consume(k, t0);
    }
  }
}

// The wave's final (m, l) of the heads its o rows hold: Me[e] / Le[e] for head
// 4g + e (l summed over the 4 row groups of token slots).
__device__ __forceinline__ void mfma_finish(const MfmaState& st, int g, float (&Me)[4],
                                            float (&Le)[4]) {
  const float L = xor32_sum(xor16_sum(st.lsum));
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    Me[e] = __shfl(st.m, 4 * g + e, 64);
    Le[e] = __shfl(L, 4 * g + e, 64);
  }
}

}  // namespace gqa
