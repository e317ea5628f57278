// MLA absorbed-path paged decode for gfx950 (the reference's roadmap item K2,
// README.md:405-408): every query row (s_q x h_q of a request) attends over
// one shared latent cache of 576-dim rows; values are the rows' first 512
// dims. Semantics and layouts: include/mla_decode.h.
//
// Work decomposition. A workgroup of 4 waves (one per SIMD) owns 128 query
// rows of one request and one split of its tokens; each wave owns 32 rows as
// two 16-row MFMA column blocks. All rows share the cache rows, so each
// 32-token tile (36 KiB) is read from HBM once per workgroup: the waves load it
// cooperatively into registers, one tile ahead, and store it into one of two
// LDS buffers, then every wave computes from LDS.
//
// LDS tile layout ("A order"): 36 blocks of 1 KiB, block (tg, kk) for token
// group tg (16 tokens) and 32-dim k-step kk holds, at 16 * lane, the 16 bytes
// lane (j = lane % 16, g = lane / 16) needs as the A operand of
// v_mfma_f32_16x16x32_bf16: token 16 tg + j, dims 32 kk + 8 g .. +8. A wave's
// staging loads and stores fill whole blocks (contiguous 1 KiB stores), and
// the QK operand reads are contiguous too.
//
//   QK^T   S^T[16 tok x 16 rows] = K[tok x 576] . Q^T[576 x 16 rows]: 18
//          MFMAs per token group and row block; A from LDS (shared by both
//          row blocks), B = Q^T in registers (lane: row j, dims 32 kk + 8 g).
//   softmax on the C layout (lane: row j, tokens 4 g + e), base 2, fp32
//          state; P rounded to bf16, l sums the rounded values.
//   PV     O[16 rows x 512] += P[rows x 32 tok] . V[32 tok x 512]: 32
//          v_mfma_f32_16x16x32_bf16 per row block (k-slot 8g+e -> token
//          4g+e, 8g+4+e -> token 16+4g+e); B read from the same LDS tile with
//          ds_read_b64_tr_b16 (lane x of a 16-lane group supplies token
//          4g + x/4, dims 16nb + 4(x%4) .. +4; the transpose hands lane x the
//          four tokens of dim 16nb + x).
//
// Splits cut a request at multiples of 32 tokens; a merge kernel folds them
// in split order (log-sum-exp), so results are bitwise reproducible.
#include "gqa_device.hpp"
#include "gqa_launch.hpp"
#include "mla_decode.h"

#include <algorithm>

namespace mla {

using gqa::exp2_fast;
using gqa::f32_to_bf16_bits;
using gqa::FastDiv;
using gqa::kLn2;
using gqa::kLog2e;
using gqa::kNegInf;

constexpr int kD = MLA_DECODE_HEAD_DIM;     // 576
constexpr int kDV = MLA_DECODE_HEAD_DIM_V;  // 512
constexpr int kKSteps = kD / 32;            // 18 QK k-steps
constexpr int kTile = 32;                   // tokens per tile
constexpr int kWaves = 4;
constexpr int kRowsPerWave = 32;
constexpr int kRowsPerGroup = kWaves * kRowsPerWave;  // 128
constexpr int kTileBlocks = 2 * kKSteps;              // 36 blocks of 1 KiB
constexpr int kTileBytes = kTileBlocks * 1024;
constexpr int kStageLoads = kTileBlocks / kWaves;     // 9 per wave per tile
constexpr int kNB = kDV / 16;                         // 32 PV column blocks
// Q^T k-steps [0, kQLds) live in LDS (one 1 KiB block per 16-row block and
// k-step), the rest in registers: all 18 in registers would not fit next to
// the 32 x 512 fp32 accumulators.
constexpr int kQLds = 9;
constexpr int kQRegs = kKSteps - kQLds;
constexpr int kQBlocks = (kRowsPerGroup / 16) * kQLds;  // 72 blocks of 1 KiB
static_assert(kTileBlocks % kWaves == 0, "staging blocks must split evenly");

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4_t;

struct MlaArgs {
  const uint16_t* q;
  const uint16_t* kv;
  const int* block_table;
  const int* seq_lens;
  uint16_t* out;
  float* lse;
  float* ws_acc;  // [B, R, ns, 512]
  float* ws_m;    // [B, R, ns] natural-log units
  float* ws_l;
  int B, s_q, h_q, R, block_size, max_blocks, num_splits, causal;
  FastDiv bs_div;
  float scale_log2e;
};

__device__ __forceinline__ bf16x8_t as_bf16x8(const uint4& u) {
  return __builtin_bit_cast(bf16x8_t, u);
}

// One row block's running state; lane (j, g): m and lsum of row j (lsum over
// this lane's token slots only), o[nb][e] = O[row 4g + e][dim 16 nb + j].
struct RowState {
  float m, lsum;
  f32x4_t o[kNB];
};

template <bool kBlockUniform>
__global__ __launch_bounds__(256, 1) void mla_decode_kernel(const MlaArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t tiles[2][kTileBytes];
  __shared__ __attribute__((aligned(16))) uint8_t qlds[kQBlocks * 1024];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int b = blockIdx.y, split = blockIdx.z;
  const int row0 = blockIdx.x * kRowsPerGroup + w * kRowsPerWave;
  const bool active = row0 < a.R;  // wave-uniform: rows past R only help stage

  const int s_cap = a.max_blocks * a.block_size;
  const int S = min(max(a.seq_lens[b], 0), s_cap);
  const int ns = a.num_splits;
  const int chunk = ((S + ns - 1) / ns + (kTile - 1)) & ~(kTile - 1);
  const int seg_start = min(split * chunk, S);
  const int seg_end = min(S, seg_start + chunk);
  const int ntiles = (seg_end - seg_start + kTile - 1) / kTile;

  // Q^T as the B operand (lane: row j, dims 32 kk + 8 g): k-steps below kQLds
  // go to this wave's LDS blocks (2w + rb, kk), the rest stay in registers;
  // and each lane's key limit for its row j.
  uint4 qf[2][kQRegs];
  int lim[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int r = row0 + 16 * rb + j;
    const bool live = r < a.R;
    const uint16_t* qrow = a.q + ((size_t)b * a.R + (live ? r : 0)) * kD + 8 * g;
#pragma unroll
    for (int kk = 0; kk < kKSteps; ++kk) {
      const uint4 v = live ? *reinterpret_cast<const uint4*>(qrow + 32 * kk) : make_uint4(0, 0, 0, 0);
      if (kk < kQLds)
        *reinterpret_cast<uint4*>(&qlds[((2 * w + rb) * kQLds + kk) * 1024 + 16 * lane]) = v;
      else
        qf[rb][kk - kQLds] = v;
    }
    const int qi = live ? r / a.h_q : 0;
    lim[rb] = min(seg_end, a.causal ? S - (a.s_q - 1 - qi) : S);
  }

  RowState st[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    st[rb].m = kNegInf;
    st[rb].lsum = 0.f;
#pragma unroll
    for (int nb = 0; nb < kNB; ++nb) st[rb].o[nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  const int* bt = a.block_table + (size_t)b * a.max_blocks;
  // The table is read-only for the launch; through the constant address space
  // the uniform block-id loads become scalar loads.
  const __attribute__((address_space(4))) int* btc =
      (const __attribute__((address_space(4))) int*)bt;
  const int bs = a.block_size;

  // Staging: wave w loads blocks w, w + 4, ... of tile k. Tokens at or past
  // seg_end read the tile's first token instead (masked later), so nothing
  // outside the request's live cache rows is touched.
  auto stage_load = [&](int k, uint4 (&r)[kStageLoads]) {
    const int ts = seg_start + kTile * k;
#pragma unroll
    for (int i = 0; i < kStageLoads; ++i) {
      const int blk = w + kWaves * i;
      const int tg = blk / kKSteps, kk = blk - tg * kKSteps;
      const int tl = 16 * tg + j;
      size_t row;
      if constexpr (kBlockUniform) {
        // 32 tokens from a 32-aligned start share one block.
        const uint32_t lb = gqa::fastdiv((uint32_t)ts, a.bs_div);
        const int slot0 = ts - (int)lb * bs;
        row = (size_t)btc[lb] * bs + slot0 + (ts + tl < seg_end ? tl : 0);
      } else {
        const int t = ts + tl < seg_end ? ts + tl : ts;
        const uint32_t lb = gqa::fastdiv((uint32_t)t, a.bs_div);
        row = (size_t)bt[lb] * bs + (t - (int)lb * bs);
      }
      r[i] = gqa::load_kv(a.kv + row * kD + 32 * kk + 8 * g);
    }
  };
  auto stage_store = [&](int buf, const uint4 (&r)[kStageLoads]) {
#pragma unroll
    for (int i = 0; i < kStageLoads; ++i)
      *reinterpret_cast<uint4*>(&tiles[buf][(w + kWaves * i) * 1024 + 16 * lane]) = r[i];
  };

  auto consume = [&](int k, int buf) {
    if (!active) return;
    const uint8_t* T = tiles[buf];
    const int ts = seg_start + kTile * k;
    // QK^T: c[rb][tg][e] = score of token 16 tg + 4 g + e for row j of block rb.
    f32x4_t c[2][2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int tg = 0; tg < 2; ++tg) c[rb][tg] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < kKSteps; ++kk) {
      uint4 qv[2];
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
        qv[rb] = kk < kQLds ? *reinterpret_cast<const uint4*>(
                                  &qlds[((2 * w + rb) * kQLds + kk) * 1024 + 16 * lane])
                            : qf[rb][kk - kQLds];
#pragma unroll
      for (int tg = 0; tg < 2; ++tg) {
        const uint4 kf = *reinterpret_cast<const uint4*>(T + (tg * kKSteps + kk) * 1024 + 16 * lane);
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
          c[rb][tg] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kf), as_bf16x8(qv[rb]),
                                                              c[rb][tg], 0, 0, 0);
      }
      // Keep the operand reads of at most two k-steps ahead of their MFMAs:
      // hoisting all of them would take more registers than the wave has.
      if (kk & 1) __builtin_amdgcn_sched_barrier(0);
    }

    uint32_t pw[2][4];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      float s[2][4];
      float mx = kNegInf;
#pragma unroll
      for (int tg = 0; tg < 2; ++tg)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool valid = ts + 16 * tg + 4 * g + e < lim[rb];
          s[tg][e] = valid ? c[rb][tg][e] * a.scale_log2e : kNegInf;
          mx = fmaxf(mx, s[tg][e]);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mn = fmaxf(st[rb].m, mx);
      const float ms = mn == kNegInf ? 0.f : mn;
      const float alpha = exp2_fast(st[rb].m - ms);
      st[rb].m = mn;
      float psum = 0.f;
#pragma unroll
      for (int tg = 0; tg < 2; ++tg)
#pragma unroll
        for (int e = 0; e < 4; e += 2) {
          const gqa::bf16x2_t pb = __builtin_convertvector(
              (float __attribute__((ext_vector_type(2)))){exp2_fast(s[tg][e] - ms),
                                                          exp2_fast(s[tg][e + 1] - ms)},
              gqa::bf16x2_t);
          const uint32_t wd = __builtin_bit_cast(uint32_t, pb);
          pw[rb][2 * tg + e / 2] = wd;
          psum += gqa::bf16_lo(wd) + gqa::bf16_hi(wd);
        }
      st[rb].lsum = fmaf(st[rb].lsum, alpha, psum);
      // Rescale O rows (4g + e) when any row's max moved.
      if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
        float ae[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) ae[e] = __shfl(alpha, 4 * g + e, 64);
#pragma unroll
        for (int nb = 0; nb < kNB; ++nb)
#pragma unroll
          for (int e = 0; e < 4; ++e) st[rb].o[nb][e] *= ae[e];
      }
    }

    // PV. Lane (j, g) supplies token 4g + j/4 (and 16 more), dims
    // 16nb + 4(j%4) .. +4 of the A-order tile.
    const int rr = 4 * g + (j >> 2);
#pragma unroll
    for (int nb = 0; nb < kNB; ++nb) {
      const int kk = nb >> 1;
      const int gg = 2 * (nb & 1) + ((j & 3) >> 1);
      const uint32_t off = (uint32_t)kk * 1024 + 16u * (uint32_t)(rr + 16 * gg) + 8u * (j & 1);
      const bf16x4_t v0 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t*)(T + off));
      const bf16x4_t v1 =
          __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t*)(T + off + kKSteps * 1024));
      const bf16x8_t vb = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        const bf16x8_t pa =
            as_bf16x8(make_uint4(pw[rb][0], pw[rb][1], pw[rb][2], pw[rb][3]));
        st[rb].o[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, vb, st[rb].o[nb], 0, 0, 0);
      }
      if (nb & 1) __builtin_amdgcn_sched_barrier(0);
    }
  };

  if (ntiles > 0) {
    uint4 r[kStageLoads];
    stage_load(0, r);
    stage_store(0, r);
    __syncthreads();
    for (int k = 0; k < ntiles; ++k) {
      const int buf = k & 1;
      if (k + 1 < ntiles) stage_load(k + 1, r);
      consume(k, buf);
      if (k + 1 < ntiles) stage_store(buf ^ 1, r);
      __syncthreads();
    }
  }
  if (!active) return;

  // Final (m, l) of the rows this lane's o entries hold: rows 4g + e.
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    float L = st[rb].lsum + __shfl_xor(st[rb].lsum, 16, 64);
    L += __shfl_xor(L, 32, 64);
    float Me[4], Le[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      Me[e] = __shfl(st[rb].m, 4 * g + e, 64);
      Le[e] = __shfl(L, 4 * g + e, 64);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = row0 + 16 * rb + 4 * g + e;
      if (row >= a.R) continue;
      const size_t br = (size_t)b * a.R + row;
      if (ns == 1) {
        const float inv = Le[e] > 0.f ? 1.f / Le[e] : 0.f;
#pragma unroll
        for (int nb = 0; nb < kNB; ++nb)
          a.out[br * kDV + 16 * nb + j] = (uint16_t)f32_to_bf16_bits(st[rb].o[nb][e] * inv);
        if (a.lse && j == 0) {
          const int qi = row / a.h_q, h = row - qi * a.h_q;
          a.lse[((size_t)b * a.h_q + h) * a.s_q + qi] =
              Le[e] > 0.f ? Me[e] * kLn2 + logf(Le[e]) : kNegInf;
        }
      } else {
        const size_t sx = br * ns + split;
#pragma unroll
        for (int nb = 0; nb < kNB; ++nb) a.ws_acc[sx * kDV + 16 * nb + j] = st[rb].o[nb][e];
        if (j == 0) {
          a.ws_m[sx] = Me[e] == kNegInf ? kNegInf : Me[e] * kLn2;  // natural-log units
          a.ws_l[sx] = Le[e];
        }
      }
    }
  }
}

// Log-sum-exp merge of the splits of each (request, query row) in split order:
// one wave per row, lane i owns dims 8i .. 8i + 8.
__global__ __launch_bounds__(256) void mla_decode_merge_kernel(const MlaArgs a) {
  constexpr int kBatch = 8;
  const int lane = threadIdx.x & 63;
  const size_t br = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (br >= (size_t)a.B * a.R) return;
  const int ns = a.num_splits;
  const size_t st0 = br * ns;
  float mloc = kNegInf;
  for (int i = lane; i < ns; i += 64) mloc = fmaxf(mloc, a.ws_m[st0 + i]);
  const float M = gqa::wave_max(mloc);
  float L = 0.f, A[8];
#pragma unroll
  for (int d = 0; d < 8; ++d) A[d] = 0.f;
  if (M != kNegInf) {
    for (int i0 = 0; i0 < ns; i0 += kBatch) {
      float mi[kBatch], li[kBatch];
      float4 a0[kBatch], a1[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const size_t sx = st0 + min(i0 + k, ns - 1);  // past the end: a valid split, not folded
        mi[k] = a.ws_m[sx];
        li[k] = a.ws_l[sx];
        const float4* src = reinterpret_cast<const float4*>(a.ws_acc + sx * kDV + 8 * lane);
        a0[k] = src[0];
        a1[k] = src[1];
      }
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        if (i0 + k >= ns) break;
        // Exactly 1 for the split holding the max; 0 for empty splits.
        const float f = mi[k] == M ? 1.f : exp2_fast((mi[k] - M) * kLog2e);
        const float av[8] = {a0[k].x, a0[k].y, a0[k].z, a0[k].w, a1[k].x, a1[k].y, a1[k].z, a1[k].w};
        L = fmaf(li[k], f, L);
#pragma unroll
        for (int d = 0; d < 8; ++d) A[d] = fmaf(av[d], f, A[d]);
      }
    }
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  uint32_t wv[4];
#pragma unroll
  for (int d = 0; d < 4; ++d)
    wv[d] = f32_to_bf16_bits(A[2 * d] * inv) | (f32_to_bf16_bits(A[2 * d + 1] * inv) << 16);
  *reinterpret_cast<uint4*>(a.out + br * kDV + 8 * lane) = make_uint4(wv[0], wv[1], wv[2], wv[3]);
  if (a.lse && lane == 0) {
    const int b = (int)(br / a.R), row = (int)(br - (size_t)b * a.R);
    const int qi = row / a.h_q, h = row - qi * a.h_q;
    a.lse[((size_t)b * a.h_q + h) * a.s_q + qi] = L > 0.f ? M + logf(L) : kNegInf;
  }
}

}  // namespace mla

extern "C" size_t mla_decode_workspace_bytes(int B, int s_q, int h_q, int num_splits) {
  if (B <= 0 || s_q <= 0 || h_q <= 0 || num_splits <= 1) return 0;
  return (size_t)B * s_q * h_q * num_splits * (mla::kDV + 2) * sizeof(float);
}

extern "C" int mla_decode_pick_num_splits(int B, int s_q, int h_q, int block_size, int max_blocks,
                                          int num_cus) {
  constexpr int64_t kMinChunk = 256;
  if (B < 1 || s_q < 1 || h_q < 1 || block_size < 1 || max_blocks < 1) return 0;
  if (num_cus <= 0 && (num_cus = gqa::device_cu_count()) <= 0) return 0;
  const int64_t groups = (int64_t)B * ((int64_t)s_q * h_q + mla::kRowsPerGroup - 1) /
                         mla::kRowsPerGroup;
  int64_t ns = (num_cus + groups - 1) / groups;
  const int64_t s_max = (int64_t)max_blocks * block_size;
  ns = std::min<int64_t>(ns, std::max<int64_t>(1, s_max / kMinChunk));
  ns = std::min<int64_t>(ns, MLA_DECODE_MAX_SPLITS);
  return (int)std::max<int64_t>(ns, 1);
}

extern "C" int mla_decode_launch(const uint16_t* q, const uint16_t* kv_cache, const int* block_table,
                                 const int* seq_lens, uint16_t* out, float* lse, int B, int s_q,
                                 int h_q, int block_size, int max_blocks, float scale, int causal,
                                 int num_splits, void* workspace, size_t workspace_bytes,
                                 hipStream_t stream) {
  if (B < 0 || B > 65535 || s_q < 1 || h_q < 1 || block_size < 1 || max_blocks < 1)
    return hipErrorInvalidValue;
  const int64_t R = (int64_t)s_q * h_q;
  if (R > (int64_t(1) << 20) || (int64_t)B * R > (int64_t(1) << 31)) return hipErrorInvalidValue;
  if ((int64_t)block_size * max_blocks >= (int64_t(1) << 31)) return hipErrorInvalidValue;
  if (num_splits < 1 || num_splits > MLA_DECODE_MAX_SPLITS) return hipErrorInvalidValue;
  if (B == 0) return hipSuccess;
  if (!q || !kv_cache || !block_table || !seq_lens || !out) return hipErrorInvalidValue;
  mla::MlaArgs a;
  a.q = q;
  a.kv = kv_cache;
  a.block_table = block_table;
  a.seq_lens = seq_lens;
  a.out = out;
  a.lse = lse;
  a.ws_acc = a.ws_m = a.ws_l = nullptr;
  a.B = B;
  a.s_q = s_q;
  a.h_q = h_q;
  a.R = (int)R;
  a.block_size = block_size;
  a.max_blocks = max_blocks;
  a.num_splits = num_splits;
  a.causal = causal ? 1 : 0;
  a.bs_div = gqa::make_fastdiv((uint32_t)block_size);
  a.scale_log2e = (float)((double)scale * 1.4426950408889634);
  if (num_splits > 1) {
    if (!workspace || ((uintptr_t)workspace & 15) != 0 ||
        workspace_bytes < mla_decode_workspace_bytes(B, s_q, h_q, num_splits))
      return hipErrorInvalidValue;
    const size_t states = (size_t)B * R * num_splits;
    a.ws_acc = static_cast<float*>(workspace);
    a.ws_m = a.ws_acc + states * mla::kDV;
    a.ws_l = a.ws_m + states;
  }
  const dim3 grid((unsigned)((R + mla::kRowsPerGroup - 1) / mla::kRowsPerGroup), B, num_splits);
  if (block_size % mla::kTile == 0)
    hipLaunchKernelGGL(mla::mla_decode_kernel<true>, grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(mla::mla_decode_kernel<false>, grid, dim3(256), 0, stream, a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || num_splits == 1) return err;
  const size_t rows = (size_t)B * R;
  hipLaunchKernelGGL(mla::mla_decode_merge_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                     stream, a);
  return hipGetLastError();
}
