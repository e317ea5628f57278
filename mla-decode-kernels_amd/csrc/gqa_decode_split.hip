// v1 (single pass) and v2 (split-KV partial + log-sum-exp merge) decode
// kernels for gfx950.
//
// Work decomposition. A workgroup of P wave64s owns one kv-head of one request
// (and one split in v2) and serves every q-head of its GQA group from the same
// K/V registers, so each K/V row crosses HBM once (the reference's per-q-head
// CTAs rely on L2 for that: kernels/gqa_decode/v2_splitkv.cu:18-24). The P
// waves deal the segment's 16-token tiles round-robin. The 64 lanes of a wave
// form 4 DPP rows of 16 lanes; a row reads one 256-byte K (or V) head row with
// 16-byte loads, so one load instruction covers 4 tokens and a tile is 4 K
// loads + 4 V loads per lane.
//
// Per tile: QK^T with v_dot2c_f32_bf16 on the packed bf16 q and K words, a
// 4-step DPP row reduction, then one online-softmax update per (row, head) for
// the whole tile (max over its 4 tokens, one rescale of l and acc) in base-2
// units, and PV as fp32 FMAs. The next tile's loads are issued before the
// current tile is consumed. At the end the row states of each wave and then
// the P wave states are merged in a fixed order: bitwise deterministic.
//
// Split rule: segment `split` of request b covers
// [split*chunk, min(S, (split+1)*chunk)) with chunk = ceil(S/num_splits)
// rounded up to a multiple of 32 tokens (v2_splitkv.cu:30-32 without the
// rounding). The rounding keeps every 16-token group inside one cache block
// whenever block_size is a multiple of 16, which lets the block id be a scalar
// load, and is the same for both scan kernels.
// Splits past the end of a short request are empty and store the neutral
// state (-inf, 0, 0), whose merge factor is 0 (v2_splitkv.cu:33-40).
// num_splits == 1 runs the single-pass kernel, so v2 with one split equals v1
// bit for bit.
#include "gqa_device.hpp"
#include "gqa_launch.hpp"
#include "gqa_scan.hpp"
#include "gqa_decode.h"

namespace gqa {

constexpr int kTile = 16;   // tokens per wave per tile
constexpr int kChunkAlign = 32;  // split lengths are multiples of this (both scan kernels)
constexpr int kLoads = 4;   // 16-byte K loads (and V loads) per lane per tile

// Launch shapes. A workgroup holds P waves that share one kv-head of one
// request and split, take its 16-token tiles round-robin and merge their
// states through LDS. Measured on MI355X: the stream runs fastest with about
// one wave per SIMD resident (4 per CU), each keeping one tile in flight while
// it consumes the previous one; more resident waves or deeper prefetch only add
// queueing. P = 4 waves per kv-head keeps a workgroup's reads adjacent and the
// merge in LDS.
// GQA groups larger than this run the matrix-core scan (gqa_decode_mfma.hip):
// its VALU work per tile does not grow with the group, while this kernel's
// does (measured: 8-head groups are VALU-bound here at ~60% of HBM peak and
// reach ~72% on MFMA; 4-head groups stream ~5% faster here).
#ifndef GQA_MFMA_MIN_GROUP
#define GQA_MFMA_MIN_GROUP 5
#endif
constexpr int kWavesPerHead = 4;  // P: waves sharing a kv-head (both kernels)
constexpr int kScanDepth = 2;     // register tiles in flight per wave


struct TileRegs {
  uint4 k[kLoads];
  uint4 v[kLoads];
};

// One workgroup = P waves on one kv-head of one request b, one q-head chunk of
// GH heads and one split; wave w takes tiles w, w + P, ... of the segment.
// Single-pass launches (num_splits == 1) with `out` set write the normalised
// output; with the workspace set they write the unnormalised state (both
// when both are set).
template <int GH, int P, int DEPTH, bool kBlockUniform>
__global__ __launch_bounds__(64 * P) void gqa_decode_scan_kernel(const ScanArgs a) {
  const int lane = threadIdx.x & 63;
  const int ph = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane >> 4;  // DPP row: token 4j + r of each load j
  const int c = lane & 15;  // dims [8c, 8c + 8)
  const int hkv = blockIdx.x / a.nchunk;
  const int hc = blockIdx.x - hkv * a.nchunk;
  const int b = blockIdx.y, split = blockIdx.z;
  const int h0 = hkv * a.G + hc * GH;  // first q-head of this wave
  const int nh = min(GH, a.G - hc * GH);

  const int S = max(a.seq_lens[b], 0);
  const int ns = a.num_splits;
  const int chunk = ((S + ns - 1) / ns + (kChunkAlign - 1)) & ~(kChunkAlign - 1);
  const int seg_start = min(split * chunk, S);
  const int seg_end = min(S, seg_start + chunk);
  const int ntiles = (seg_end - seg_start + kTile - 1) / kTile;
  const int my_tiles = ntiles > ph ? (ntiles - ph + P - 1) / P : 0;

  uint4 qf[GH];
#pragma unroll
  for (int j = 0; j < GH; ++j) {
    qf[j] = make_uint4(0, 0, 0, 0);
    if (j < nh)
      qf[j] = *reinterpret_cast<const uint4*>(a.q + ((size_t)b * a.Hq + h0 + j) * kHeadDim + 8 * c);
  }

  float m[GH], l[GH], acc[GH][8];
#pragma unroll
  for (int j = 0; j < GH; ++j) {
    m[j] = kNegInf;
    l[j] = 0.f;
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[j][d] = 0.f;
  }

  const uint32_t row_elems = (uint32_t)a.Hkv * kHeadDim;  // elements between slots
  const uint16_t* kbase = a.k_cache + (size_t)hkv * kHeadDim + 8 * c;
  const uint16_t* vbase = a.v_cache + (size_t)hkv * kHeadDim + 8 * c;
  const int* bt = a.block_table + (size_t)b * a.max_blocks;
  const int bs = a.block_size;

  auto tile_start = [&](int k) { return seg_start + kTile * (ph + P * k); };

  // Issue the K and V loads of this wave's tile k. Tokens at or past seg_end
  // read the tile's first token instead (always valid), so no load touches an
  // unallocated block or a tail slot; their scores are masked in consume().
  auto issue = [&](int k, TileRegs& t) {
    const int ts = tile_start(k);
    if constexpr (kBlockUniform) {
      // The 16 tokens of the tile share one block: scalar block-id load, a
      // uniform 64-bit block base and 32-bit per-lane offsets inside it.
      const uint32_t lb = fastdiv((uint32_t)ts, a.bs_div);
      const int slot0 = ts - (int)lb * bs;
      const size_t blk = (size_t)bt[lb] * ((size_t)bs * row_elems) + (size_t)hkv * kHeadDim;
      const uint16_t* kblk = a.k_cache + blk;
      const uint16_t* vblk = a.v_cache + blk;
#pragma unroll
      for (int j = 0; j < kLoads; ++j) {
        const int tok = ts + 4 * j + r;
        const uint32_t slot = tok < seg_end ? slot0 + 4 * j + r : slot0;
        const uint32_t off = slot * row_elems + 8 * c;
        t.k[j] = *reinterpret_cast<const uint4*>(kblk + off);
        t.v[j] = *reinterpret_cast<const uint4*>(vblk + off);
      }
    } else {
#pragma unroll
      for (int j = 0; j < kLoads; ++j) {
        int tok = ts + 4 * j + r;
        tok = tok < seg_end ? tok : ts;
        const uint32_t lb = fastdiv((uint32_t)tok, a.bs_div);
        const int slot = tok - (int)lb * bs;
        const size_t off = ((size_t)bt[lb] * bs + slot) * row_elems;
        t.k[j] = *reinterpret_cast<const uint4*>(kbase + off);
        t.v[j] = *reinterpret_cast<const uint4*>(vbase + off);
      }
    }
  };

  auto consume = [&](int k, const TileRegs& t) {
    const int ts = tile_start(k);
    float s[kLoads][GH];  // scores (base-2 units), then probabilities
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
      const bool valid = ts + 4 * j + r < seg_end;
#pragma unroll
      for (int h = 0; h < GH; ++h) {
        float d = dot2_bf16(qf[h].x, t.k[j].x, 0.f);
        d = dot2_bf16(qf[h].y, t.k[j].y, d);
        d = dot2_bf16(qf[h].z, t.k[j].z, d);
        d = dot2_bf16(qf[h].w, t.k[j].w, d);
        d = row16_sum(d);
        s[j][h] = valid ? d * a.scale_log2e : kNegInf;
      }
    }
#pragma unroll
    for (int h = 0; h < GH; ++h) {
      const float mt = fmaxf(fmaxf(s[0][h], s[1][h]), fmaxf(s[2][h], s[3][h]));
      const float mn = fmaxf(m[h], mt);
      const float ms = mn == kNegInf ? 0.f : mn;  // a row with no valid token yet
      const float al = exp2_fast(m[h] - ms);
      m[h] = mn;
#pragma unroll
      for (int j = 0; j < kLoads; ++j) s[j][h] = exp2_fast(s[j][h] - ms);
      l[h] = fmaf(l[h], al, (s[0][h] + s[1][h]) + (s[2][h] + s[3][h]));
#pragma unroll
      for (int d = 0; d < 8; ++d) acc[h][d] *= al;
    }
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
      const float vf[8] = {bf16_lo(t.v[j].x), bf16_hi(t.v[j].x), bf16_lo(t.v[j].y),
                           bf16_hi(t.v[j].y), bf16_lo(t.v[j].z), bf16_hi(t.v[j].z),
                           bf16_lo(t.v[j].w), bf16_hi(t.v[j].w)};
#pragma unroll
      for (int h = 0; h < GH; ++h)
#pragma unroll
        for (int d = 0; d < 8; ++d) acc[h][d] = fmaf(s[j][h], vf[d], acc[h][d]);
    }
  };

  // DEPTH register tiles in flight. The steady-state loop body issues tile
  // k + DEPTH - 1 before consuming tile k and has no branch, so the wait before
  // each consume covers only the tile being consumed.
  if (my_tiles > 0) {
    TileRegs t[DEPTH];
#pragma unroll
    for (int i = 0; i < DEPTH - 1; ++i)
      if (i < my_tiles) issue(i, t[i]);
    int k = 0;
    for (; k + 2 * DEPTH - 2 < my_tiles; k += DEPTH) {
#pragma unroll
      for (int i = 0; i < DEPTH; ++i) {
        issue(k + i + DEPTH - 1, t[(i + DEPTH - 1) % DEPTH]);
        consume(k + i, t[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < DEPTH; ++i) {
      if (k + i < my_tiles) {
        if (k + i + DEPTH - 1 < my_tiles) issue(k + i + DEPTH - 1, t[(i + DEPTH - 1) % DEPTH]);
        consume(k + i, t[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < DEPTH - 1; ++i) {
      // At most 2*DEPTH - 2 tiles remain after the loop; the block above
      // consumed DEPTH of them.
      if (k + DEPTH + i < my_tiles) {
        if (k + DEPTH + i + DEPTH - 1 < my_tiles)
          issue(k + DEPTH + i + DEPTH - 1, t[(i + 2 * DEPTH - 1) % DEPTH]);
        consume(k + DEPTH + i, t[(DEPTH + i) % DEPTH]);
      }
    }
  }

  // Merge the 4 row states of the wave (every row ends with the same totals).
  float Mw[GH], Lw[GH];
#pragma unroll
  for (int h = 0; h < GH; ++h) {
    const float mr = m[h];
    float M = fmaxf(mr, __shfl_xor(mr, 16, 64));
    M = fmaxf(M, __shfl_xor(M, 32, 64));
    const float f = mr == M ? 1.f : exp2_fast(mr - (M == kNegInf ? 0.f : M));
    float lr = l[h] * f;
    lr += __shfl_xor(lr, 16, 64);
    lr += __shfl_xor(lr, 32, 64);
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      float x = acc[h][d] * f;
      x += __shfl_xor(x, 16, 64);
      x += __shfl_xor(x, 32, 64);
      acc[h][d] = x;
    }
    Mw[h] = M;
    Lw[h] = lr;
  }

  if constexpr (P == 1) {
    // The wave holds the whole state of its kv-head: row 0 writes it.
    if (r == 0) {
#pragma unroll
      for (int h = 0; h < GH; ++h) {
        if (h >= nh) continue;
        const size_t bh = (size_t)b * a.Hq + h0 + h;
        if (a.out) {
          uint32_t w[4];
#pragma unroll
          for (int d = 0; d < 4; ++d)
            w[d] = f32_to_bf16_bits(finalize(acc[h][2 * d], Lw[h])) |
                   (f32_to_bf16_bits(finalize(acc[h][2 * d + 1], Lw[h])) << 16);
          *reinterpret_cast<uint4*>(a.out + bh * kHeadDim + 8 * c) = make_uint4(w[0], w[1], w[2], w[3]);
        }
        if (a.ws_acc) {
          const size_t st = bh * ns + split;
          float4* dst = reinterpret_cast<float4*>(a.ws_acc + st * kHeadDim + 8 * c);
          dst[0] = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
          dst[1] = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
          if (c == 0) {
            a.ws_m[st] = Mw[h] * kLn2;  // back to natural-log units
            a.ws_l[st] = Lw[h];
          }
        }
      }
    }
  } else {
    // P waves share the kv-head: merge their states through LDS in wave order.
    __shared__ float lds_m[P][GH];
    __shared__ float lds_l[P][GH];
    __shared__ float lds_acc[P][GH][kHeadDim];
#pragma unroll
    for (int h = 0; h < GH; ++h) {
      if (r == 0) {
        float4* dst = reinterpret_cast<float4*>(&lds_acc[ph][h][8 * c]);
        dst[0] = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
        dst[1] = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
      }
      if (lane == 0) {
        lds_m[ph][h] = Mw[h];
        lds_l[ph][h] = Lw[h];
      }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < nh * kHeadDim; idx += 64 * P) {
      const int h = idx / kHeadDim, d = idx % kHeadDim;
      float M = lds_m[0][h];
#pragma unroll
      for (int w = 1; w < P; ++w) M = fmaxf(M, lds_m[w][h]);
      const float Ms = M == kNegInf ? 0.f : M;
      float L = 0.f, A = 0.f;
#pragma unroll
      for (int w = 0; w < P; ++w) {
        const float mw = lds_m[w][h];
        const float f = mw == M ? 1.f : exp2_fast(mw - Ms);
        if (w == 0) {
          L = lds_l[0][h] * f;
          A = lds_acc[0][h][d] * f;
        } else {
          L = fmaf(lds_l[w][h], f, L);
          A = fmaf(lds_acc[w][h][d], f, A);
        }
      }
      const size_t bh = (size_t)b * a.Hq + h0 + h;
      if (a.out) a.out[bh * kHeadDim + d] = (uint16_t)f32_to_bf16_bits(finalize(A, L));
      if (a.ws_acc) {
        const size_t st = bh * ns + split;
        a.ws_acc[st * kHeadDim + d] = A;
        if (d == 0) {
          a.ws_m[st] = M * kLn2;  // back to natural-log units
          a.ws_l[st] = L;
        }
      }
    }
  }
}

// Log-sum-exp merge of the num_splits states of each (b, q-head) in split order
// (v2_splitkv.cu:92-108): one wave per (b, q-head), lane i owns dims 2i, 2i+1.
__global__ __launch_bounds__(256) void gqa_decode_merge_kernel(const float* __restrict__ ws_acc,
                                                               const float* __restrict__ ws_m,
                                                               const float* __restrict__ ws_l,
                                                               uint16_t* __restrict__ out, int BH,
                                                               int ns) {
  const int bh = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (bh >= BH) return;
  const size_t st0 = (size_t)bh * ns;
  float M = kNegInf;
  for (int i = 0; i < ns; ++i) M = fmaxf(M, ws_m[st0 + i]);
  float L = 0.f, A0 = 0.f, A1 = 0.f;
  for (int i = 0; i < ns; ++i) {
    const float mi = ws_m[st0 + i];
    // Exactly 1 for the split holding the max, so one split is a no-op merge.
    const float f = mi == M ? 1.f : exp2_fast((mi - M) * kLog2e);
    const float2 av = reinterpret_cast<const float2*>(ws_acc + (st0 + i) * kHeadDim)[lane];
    if (i == 0) {
      L = ws_l[st0] * f;
      A0 = av.x * f;
      A1 = av.y * f;
    } else {
      L = fmaf(ws_l[st0 + i], f, L);
      A0 = fmaf(av.x, f, A0);
      A1 = fmaf(av.y, f, A1);
    }
  }
  const uint32_t lo = f32_to_bf16_bits(finalize(A0, L));
  const uint32_t hi = f32_to_bf16_bits(finalize(A1, L));
  reinterpret_cast<uint32_t*>(out + (size_t)bh * kHeadDim)[lane] = lo | (hi << 16);
}

// q-heads served per wave of this kernel: the whole group (at most 4 here),
// rounded up to a power of two; extra heads carry q = 0 and are not written.
inline int heads_per_wave(int G) { return G <= 1 ? 1 : G <= 2 ? 2 : 4; }
inline bool use_mfma(int G) { return G >= GQA_MFMA_MIN_GROUP; }

template <int GH, int P>
hipError_t launch_scan_shape(const ScanArgs& a, dim3 grid, hipStream_t stream) {
  if (a.block_size % kTile == 0)
    hipLaunchKernelGGL((gqa_decode_scan_kernel<GH, P, kScanDepth, true>), grid, dim3(64 * P), 0,
                       stream, a);
  else
    hipLaunchKernelGGL((gqa_decode_scan_kernel<GH, P, kScanDepth, false>), grid, dim3(64 * P), 0,
                       stream, a);
  return hipGetLastError();
}

template <int GH>
hipError_t launch_scan_gh(const ScanArgs& a, int B, hipStream_t stream) {
  const dim3 grid(a.Hkv * a.nchunk, B, a.num_splits);
  return launch_scan_shape<GH, kWavesPerHead>(a, grid, stream);
}

hipError_t launch_scan(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                       const int* block_table, const int* seq_lens, uint16_t* out, float* ws_acc,
                       float* ws_m, float* ws_l, int B, int Hq, int Hkv, int block_size,
                       int max_blocks, float scale, int num_splits, hipStream_t stream) {
  ScanArgs a;
  a.q = q;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.block_table = block_table;
  a.seq_lens = seq_lens;
  a.out = out;
  a.ws_acc = ws_acc;
  a.ws_m = ws_m;
  a.ws_l = ws_l;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.G = Hq / Hkv;
  const int GH = heads_per_wave(a.G);
  a.nchunk = (a.G + GH - 1) / GH;
  a.block_size = block_size;
  a.max_blocks = max_blocks;
  a.num_splits = num_splits;
  a.bs_div = make_fastdiv((uint32_t)block_size);
  a.scale_log2e = (float)((double)scale * 1.4426950408889634);
  if (use_mfma(a.G)) return launch_scan_mfma(a, B, stream);
  switch (GH) {
    case 1: return launch_scan_gh<1>(a, B, stream);
    case 2: return launch_scan_gh<2>(a, B, stream);
    default: return launch_scan_gh<4>(a, B, stream);
  }
}

}  // namespace gqa

extern "C" int gqa_decode_v1_launch(const uint16_t* q, const uint16_t* k_cache,
                                    const uint16_t* v_cache, const int* block_table,
                                    const int* seq_lens, uint16_t* out, int B, int Hq, int Hkv,
                                    int block_size, int max_blocks, float scale,
                                    hipStream_t stream) {
  hipError_t err = gqa::check_common(q, k_cache, v_cache, block_table, seq_lens, out, B, Hq, Hkv,
                                     block_size, max_blocks);
  if (err != hipSuccess) return err;
  if (B == 0) return hipSuccess;
  return gqa::launch_scan(q, k_cache, v_cache, block_table, seq_lens, out, nullptr, nullptr,
                          nullptr, B, Hq, Hkv, block_size, max_blocks, scale, 1, stream);
}

extern "C" int gqa_decode_v2_partial_launch(const uint16_t* q, const uint16_t* k_cache,
                                            const uint16_t* v_cache, const int* block_table,
                                            const int* seq_lens, int B, int Hq, int Hkv,
                                            int block_size, int max_blocks, float scale,
                                            int num_splits, float* ws_acc, float* ws_m,
                                            float* ws_l, hipStream_t stream) {
  // `out` is not used by the partial kernel; pass ws_acc to the shared check.
  hipError_t err = gqa::check_common(q, k_cache, v_cache, block_table, seq_lens, ws_acc, B, Hq,
                                     Hkv, block_size, max_blocks);
  if (err != hipSuccess) return err;
  if (num_splits < 1 || num_splits > GQA_DECODE_MAX_SPLITS) return hipErrorInvalidValue;
  if (B > 0 && (!ws_acc || !ws_m || !ws_l)) return hipErrorInvalidValue;
  if (B == 0) return hipSuccess;
  return gqa::launch_scan(q, k_cache, v_cache, block_table, seq_lens, nullptr, ws_acc, ws_m, ws_l,
                          B, Hq, Hkv, block_size, max_blocks, scale, num_splits, stream);
}

extern "C" int gqa_decode_v2_merge_launch(const float* ws_acc, const float* ws_m,
                                          const float* ws_l, uint16_t* out, int B, int Hq,
                                          int num_splits, hipStream_t stream) {
  if (B < 0 || Hq < 1 || (int64_t)B * Hq > (int64_t(1) << 30)) return hipErrorInvalidValue;
  if (num_splits < 1 || num_splits > GQA_DECODE_MAX_SPLITS) return hipErrorInvalidValue;
  if (B > 0 && (!ws_acc || !ws_m || !ws_l || !out)) return hipErrorInvalidValue;
  if (B == 0) return hipSuccess;
  const int BH = B * Hq;
  hipLaunchKernelGGL(gqa::gqa_decode_merge_kernel, dim3((BH + 3) / 4), dim3(256), 0, stream,
                     ws_acc, ws_m, ws_l, out, BH, num_splits);
  return hipGetLastError();
}

extern "C" int gqa_decode_v2_launch(const uint16_t* q, const uint16_t* k_cache,
                                    const uint16_t* v_cache, const int* block_table,
                                    const int* seq_lens, uint16_t* out, int B, int Hq, int Hkv,
                                    int block_size, int max_blocks, float scale, int num_splits,
                                    float* ws_acc, float* ws_m, float* ws_l, hipStream_t stream) {
  if (B > 0 && !out) return hipErrorInvalidValue;
  if (num_splits == 1) {
    // One split: the single-pass kernel writes the output and the (one-split)
    // workspace state itself; the merge would be an exact no-op.
    hipError_t err = gqa::check_common(q, k_cache, v_cache, block_table, seq_lens, out, B, Hq, Hkv,
                                       block_size, max_blocks);
    if (err != hipSuccess) return err;
    if (B > 0 && (!ws_acc || !ws_m || !ws_l)) return hipErrorInvalidValue;
    if (B == 0) return hipSuccess;
    return gqa::launch_scan(q, k_cache, v_cache, block_table, seq_lens, out, ws_acc, ws_m, ws_l,
                            B, Hq, Hkv, block_size, max_blocks, scale, 1, stream);
  }
  const int err = gqa_decode_v2_partial_launch(q, k_cache, v_cache, block_table, seq_lens, B, Hq,
                                               Hkv, block_size, max_blocks, scale, num_splits,
                                               ws_acc, ws_m, ws_l, stream);
  if (err != hipSuccess) return err;
  return gqa_decode_v2_merge_launch(ws_acc, ws_m, ws_l, out, B, Hq, num_splits, stream);
}

extern "C" size_t gqa_decode_v2_workspace_bytes(int B, int Hq, int num_splits) {
  if (B <= 0 || Hq <= 0 || num_splits <= 0) return 0;
  return (size_t)B * Hq * num_splits * (gqa::kHeadDim + 2) * sizeof(float);
}

// Number of splits. Two bounds, the larger wins:
//  * fill: as many waves as fit in one round of the target residency -- one
//    wave per SIMD (4 per CU), or two for the matrix-core scan on long
//    sequences, whose per-tile dependency chain needs a second wave per SIMD
//    to hide -- rounded down: a round that is even slightly over-full leaves
//    its excess waves to run alone afterwards (measured: 8 requests of 32768
//    tokens take 182 us at 1024 waves, 246 us at 1280);
//  * length: no split longer than kMaxChunk tokens, so one long request in a
//    ragged batch cannot leave a tail of a few waves streaming alone;
// and two caps: each wave keeps at least kMinTilesPerWave tiles, and at most
// kMaxSplits splits (the merge walks the splits of a head in order, so very
// many short splits cost more to merge than they gain). The longest request
// is taken as max_blocks * block_size, the only length the host knows without
// reading seq_lens back from the device.
extern "C" int gqa_decode_pick_num_splits(int B, int Hq, int Hkv, int block_size, int max_blocks,
                                          int num_cus) {
  constexpr int kMinTilesPerWave = 2;
  constexpr int64_t kMaxChunk = 8192;
  constexpr int64_t kLongSequence = 8192;
  constexpr int64_t kMaxSplits = 32;
  if (B < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv != 0 || block_size < 1 || max_blocks < 1) return 0;
  if (num_cus <= 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&num_cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        num_cus <= 0)
      return 0;
  }
  const int G = Hq / Hkv;
  const bool mfma = gqa::use_mfma(G);
  const int GH = mfma ? 16 : gqa::heads_per_wave(G);  // q-heads per wave
  const int P = gqa::kWavesPerHead;
  const int64_t s_max = (int64_t)max_blocks * block_size;
  const int waves_per_cu = (mfma && s_max >= kLongSequence) ? 8 : 4;
  const int64_t waves1 = (int64_t)B * Hkv * ((G + GH - 1) / GH) * P;
  const int64_t target = (int64_t)num_cus * waves_per_cu;
  int64_t ns = target / waves1;
  const int64_t ns_len = (s_max + kMaxChunk - 1) / kMaxChunk;
  if (ns < ns_len) ns = ns_len;
  const int64_t min_chunk = (int64_t)gqa::kTile * P * kMinTilesPerWave;
  const int64_t ns_cap = s_max / min_chunk > 1 ? s_max / min_chunk : 1;
  if (ns > ns_cap) ns = ns_cap;
  if (ns > kMaxSplits) ns = kMaxSplits;
  return ns < 1 ? 1 : (int)ns;
}
