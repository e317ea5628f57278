// v1 (single pass) and v2 (split-KV partial + log-sum-exp merge) decode
// kernels for gfx950.
//
// Work decomposition. A workgroup of P wave64s owns one kv-head of one request
// (and one split in v2) and serves every q-head of its GQA group from the same
// K/V registers, so each K/V row crosses HBM once (the reference's per-q-head
// CTAs rely on L2 for that: kernels/gqa_decode/v2_splitkv.cu:18-24). The P
// waves deal the segment's 16-token tiles round-robin; the per-tile work is
// the VALU scan of gqa_scan_valu.hpp. At the end the row states of each wave
// and then the P wave states are merged in a fixed order: bitwise
// deterministic.
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
//
// Two layouts for split mode. With few splits, P waves share each split (the
// decomposition above, grid (kv-heads, B, num_splits)): 4, or 8, 12 or 16 on
// grids that leave CUs idle (waves_per_split in gqa_scan.hpp). With at least
// as many splits as one round of one wave per SIMD gives each (request,
// kv-head) waves, every split is scanned by one wave, and each wave walks a
// contiguous run of splits with one tile pipeline
// (gqa_decode_split_range_kernel): the grid stays at the single pass's size
// whatever the split count, and the splits' states are staged in LDS and
// leave after the wave's last tile. A split's state is then the sequential
// fold of its tiles, which does not depend on which wave scans it or on how
// many splits that wave takes. Grids that leave CUs idle with splits of at
// most 1024 tokens run the matrix-core scan instead (use_mfma_underfilled).
#include "gqa_device.hpp"
#include "gqa_launch.hpp"
#include "gqa_merge.hpp"
#include "gqa_scan.hpp"
#include "gqa_scan_valu.hpp"
#include "gqa_decode.h"

#include <algorithm>

namespace gqa {

// Row 0 of a wave holds the wave's merged state after merge_rows: store it as
// split `split`'s state of q-heads bh0 .. bh0 + nh - 1 (acc as 16-byte
// stores, m back in natural-log units, l), at device scope when the launch
// merges in-kernel.
template <int GH>
__device__ __forceinline__ void store_wave_state(const ScanArgs& a, size_t bh0, int nh, int split,
                                                 int r, int c, const WaveState<GH>& st,
                                                 const float (&Mw)[GH], const float (&Lw)[GH]) {
  if (r != 0) return;
#pragma unroll
  for (int h = 0; h < GH; ++h) {
    if (h >= nh) continue;
    const size_t stx = (bh0 + h) * a.num_splits + split;
    float* dst = a.ws_acc + stx * kHeadDim + 8 * c;
    if (a.counters) {
#pragma unroll
      for (int d = 0; d < 8; d += 2) store_coherent2(dst + d, st.acc[h][d], st.acc[h][d + 1]);
    } else {
      reinterpret_cast<float4*>(dst)[0] =
          make_float4(st.acc[h][0], st.acc[h][1], st.acc[h][2], st.acc[h][3]);
      reinterpret_cast<float4*>(dst)[1] =
          make_float4(st.acc[h][4], st.acc[h][5], st.acc[h][6], st.acc[h][7]);
    }
    if (c == 0) {
      put_state(a.ws_m + stx, Mw[h] * kLn2, a.counters);
      put_state(a.ws_l + stx, Lw[h], a.counters);
    }
  }
}

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
  const int hx = blockIdx.x / a.nchunk;
  const int hkv = strided_kv_head(hx, a.Hkv);
  const int hc = blockIdx.x - hx * a.nchunk;
  const int b = blockIdx.y, split = blockIdx.z;
  const int h0 = hkv * a.G + hc * GH;  // first q-head of this wave
  const int nh = min(GH, a.G - hc * GH);

  const int S = max(a.seq_lens[b], 0);
  const int ns = a.num_splits;
  const int chunk = ((S + ns - 1) / ns + (kChunkAlign - 1)) & ~(kChunkAlign - 1);
  const int seg_start = min(split * chunk, S);
  const int seg_end = min(S, seg_start + chunk);

  uint4 qf[GH];
  load_q(a, b, h0, nh, c, qf);
  WaveState<GH> st;
  init_state(st);
  scan_segment<GH, P, DEPTH, kBlockUniform>(a, a.block_table + (size_t)b * a.max_blocks, hkv, qf,
                                            seg_start, seg_end, ph, r, c, st);
  float Mw[GH], Lw[GH];
  merge_rows(st, Mw, Lw);

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
            w[d] = f32_to_bf16_bits(finalize(st.acc[h][2 * d], Lw[h])) |
                   (f32_to_bf16_bits(finalize(st.acc[h][2 * d + 1], Lw[h])) << 16);
          *reinterpret_cast<uint4*>(a.out + bh * kHeadDim + 8 * c) = make_uint4(w[0], w[1], w[2], w[3]);
        }
      }
    }
    if (a.ws_acc) store_wave_state(a, (size_t)b * a.Hq + h0, nh, split, r, c, st, Mw, Lw);
  } else {
    // P waves share the kv-head: merge their states through LDS in wave order.
    __shared__ WaveMergeLds<GH, P> lds;
    stage_wave_state(lds, ph, lane, r, c, st, Mw, Lw);
    __syncthreads();
    for (int idx = threadIdx.x; idx < nh * kHeadDim; idx += 64 * P) {
      const int h = idx / kHeadDim, d = idx % kHeadDim;
      float M, L, A;
      merge_wave_states(lds, h, d, M, L, A);
      const size_t bh = (size_t)b * a.Hq + h0 + h;
      if (a.out) a.out[bh * kHeadDim + d] = (uint16_t)f32_to_bf16_bits(finalize(A, L));
      if (a.ws_acc) {
        const size_t stx = bh * ns + split;
        put_state(a.ws_acc + stx * kHeadDim + d, A, a.counters);
        if (d == 0) {
          put_state(a.ws_m + stx, M * kLn2, a.counters);  // back to natural-log units
          put_state(a.ws_l + stx, L, a.counters);
        }
      }
    }
  }
  // Single-launch split mode: the group's last workgroup merges its (at most
  // four) heads, all in wave 0.
  if (a.counters != nullptr && arrive_last(a.counters, (size_t)b * gridDim.x + blockIdx.x, ns) &&
      ph == 0)
    merge_heads4(a.ws_acc, a.ws_m, a.ws_l, a.merge_out, (size_t)b * a.Hq + h0, nh, ns, lane);
}

// Dynamic LDS of the split-range kernel: each of its kWavesPerHead waves stages
// up to `slots` split states of its G q-heads (acc [slot][G][128], then m and l
// [slot][G][2], in floats), at most kStageBytes per workgroup (gfx950 has
// 160 KiB of LDS per CU; the rest is left for the kernel's static LDS).
constexpr int kStageBytes = 156 * 1024;
// Floats of one wave's stage of `slots` states, rounded up to 16 bytes so that
// every wave's region (and its 16-byte acc stores) stays 16-byte aligned.
__host__ __device__ constexpr int stage_wave_floats(int G, int slots) {
  return (slots * G * (kHeadDim + 2) + 3) & ~3;
}
inline int stage_cap(int G) {
  return kStageBytes / (kWavesPerHead * (G * (kHeadDim + 2) * 4 + 16));
}
inline int stage_slots(int G, int splits_per_wave) {
  return std::max(1, std::min(stage_cap(G), splits_per_wave));
}

// What the split-range kernel does with its split states.
enum class RangeMode {
  kStates,  // store them in the workspace (the partial launch)
  kArrive,  // store them at device scope; the pair's last workgroup to arrive merges
  kMerge,   // store them and merge them in the workgroup: one workgroup holds
            // all of the pair's splits in its LDS stage
};

// A wave's staged split states. stage() keeps the state of the split that just
// ended (row 0 of the wave holds it after merge_rows) in LDS: shared-memory
// stores count against a different counter than the tile loads, so the loads
// in flight are not held up by them, as they would be by global stores.
// drain() writes the staged states of splits first .. first + used - 1 to the
// workspace (each head's acc as one coalesced 512-byte store per wave; all
// LDS reads first, then the stores) and empties the stage, leaving its LDS
// contents in place; the kernel drains when the stage is full and after its
// last split.
template <int G, bool kCoherent>
struct SplitStage {
  float* acc;  // this wave's [slots][G][128]
  float* ml;   // this wave's [slots][G][2]
  int slots, used, first;

  __device__ __forceinline__ void stage(int r, int c, int lane, const WaveState<G>& st,
                                        const float (&Mw)[G], const float (&Lw)[G]) {
    if (r == 0) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float4* dst = reinterpret_cast<float4*>(acc + (used * G + h) * kHeadDim + 8 * c);
        dst[0] = make_float4(st.acc[h][0], st.acc[h][1], st.acc[h][2], st.acc[h][3]);
        dst[1] = make_float4(st.acc[h][4], st.acc[h][5], st.acc[h][6], st.acc[h][7]);
      }
    }
    if (lane < G) {
      // Lane h writes head h's m (natural-log units) and l.
      float m = Mw[0], l = Lw[0];
#pragma unroll
      for (int h = 1; h < G; ++h) {
        m = lane == h ? Mw[h] : m;
        l = lane == h ? Lw[h] : l;
      }
      *reinterpret_cast<float2*>(ml + (used * G + lane) * 2) = make_float2(m * kLn2, l);
    }
    ++used;
  }

  // The neutral state (-inf, 0, 0) of an empty split.
  __device__ __forceinline__ void stage_empty(int lane) {
#pragma unroll
    for (int h = 0; h < G; ++h)
      reinterpret_cast<float2*>(acc + (used * G + h) * kHeadDim)[lane] = make_float2(0.f, 0.f);
    if (lane < G) *reinterpret_cast<float2*>(ml + (used * G + lane) * 2) = make_float2(kNegInf, 0.f);
    ++used;
  }

  __device__ __forceinline__ void drain(const ScanArgs& a, size_t bh0, int lane) {
    const int ns = a.num_splits;
    for (int j = 0; j < used; ++j) {
      float2 v[G];
#pragma unroll
      for (int h = 0; h < G; ++h)
        v[h] = reinterpret_cast<const float2*>(acc + (j * G + h) * kHeadDim)[lane];
      // Lane h < G: head h's m and l.
      const float2 w = *reinterpret_cast<const float2*>(ml + (j * G + min(lane, G - 1)) * 2);
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const size_t stx = (bh0 + h) * ns + first + j;
        float* dst = a.ws_acc + stx * kHeadDim + 2 * lane;
        if constexpr (kCoherent)
          store_coherent2(dst, v[h].x, v[h].y);
        else
          *reinterpret_cast<float2*>(dst) = v[h];
      }
      if (lane < G) {
        const size_t stx = (bh0 + lane) * ns + first + j;
        put_state(a.ws_m + stx, w.x, kCoherent ? a.ws_m : nullptr);
        put_state(a.ws_l + stx, w.y, kCoherent ? a.ws_l : nullptr);
      }
    }
    first += used;
    used = 0;
  }
};

// Split mode with many splits, for groups of G <= 4 q-heads: a workgroup of
// kWavesPerHead waves on one kv-head of one request b, each wave serving the
// whole group. Of the W = 4 * gridDim.z waves that serve the pair, wave
// gw = 4 * blockIdx.z + ph takes the contiguous run of splits
// [gw * ns / W, (gw + 1) * ns / W) -- at least one, since the launch takes
// this layout only with ns >= W -- and scans their tokens as one range
// (scan_split_range), staging each split's state in LDS when the split ends
// (SplitStage); splits past the end of the request get the neutral state
// (-inf, 0, 0). The waves of a workgroup share nothing until the end, where,
// by kMode: they only store their states (kStates); the pair's last workgroup
// to arrive merges them from the workspace (kArrive: states stored at device
// scope); or, with one workgroup per pair whose stage holds every split, the
// workgroup merges the staged states itself, split by split in index order
// with the merge kernel's fold (kMerge: out equals partial + merge bit for
// bit, with no second launch). Dynamic LDS: kWavesPerHead regions of
// stage_wave_floats(G, slots) floats.
template <int G, bool kBlockUniform, RangeMode kMode>
__global__ __launch_bounds__(64 * kWavesPerHead) void gqa_decode_split_range_kernel(
    const ScanArgs a, int slots) {
  constexpr bool kCoherent = kMode == RangeMode::kArrive;
  extern __shared__ float4 stage_lds[];
  const int lane = threadIdx.x & 63;
  const int ph = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane >> 4;
  const int c = lane & 15;
  const int hkv = strided_kv_head(blockIdx.x, a.Hkv);
  const int b = blockIdx.y;
  const int h0 = hkv * G;
  const size_t bh0 = (size_t)b * a.Hq + h0;

  const int S = max(a.seq_lens[b], 0);
  const int ns = a.num_splits;
  const int chunk = ((S + ns - 1) / ns + (kChunkAlign - 1)) & ~(kChunkAlign - 1);
  const int W = kWavesPerHead * (int)gridDim.z;
  const int gw = kWavesPerHead * (int)blockIdx.z + ph;
  const int s_begin = (int)((int64_t)gw * ns / W);
  const int s_end = (int)((int64_t)(gw + 1) * ns / W);
  const int rs = (int)min((int64_t)s_begin * chunk, (int64_t)S);
  const int re = (int)min((int64_t)s_end * chunk, (int64_t)S);

  const int wave_floats = stage_wave_floats(G, slots);
  float* const lds = reinterpret_cast<float*>(stage_lds);
  float* wave_lds = lds + ph * wave_floats;
  SplitStage<G, kCoherent> stage{wave_lds, wave_lds + slots * G * kHeadDim, slots, 0, s_begin};

  uint4 qf[G];
  load_q(a, b, h0, G, c, qf);
  WaveState<G> st;
  init_state(st);
  scan_split_range<G, kBlockUniform>(
      a, a.block_table + (size_t)b * a.max_blocks, hkv, qf, rs, re, chunk / kTile, r, c, st,
      [&](WaveState<G>& s) {
        float Mw[G], Lw[G];
        merge_rows(s, Mw, Lw);
        stage.stage(r, c, lane, s, Mw, Lw);
        if (stage.used == stage.slots) stage.drain(a, bh0, lane);
        init_state(s);
      });
  if constexpr (kMode == RangeMode::kMerge) {
    // Every split of the wave, empty ones included, stays staged for the merge.
    while (stage.first + stage.used < s_end) stage.stage_empty(lane);
    stage.drain(a, bh0, lane);
  } else {
    stage.drain(a, bh0, lane);
    for (int split = stage.first; split < s_end; ++split) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const size_t stx = (bh0 + h) * ns + split;
        float* dst = a.ws_acc + stx * kHeadDim + 2 * lane;
        if constexpr (kCoherent)
          store_coherent2(dst, 0.f, 0.f);
        else
          *reinterpret_cast<float2*>(dst) = make_float2(0.f, 0.f);
      }
      if (lane < G) {
        const size_t stx = (bh0 + lane) * ns + split;
        put_state(a.ws_m + stx, kNegInf, kCoherent ? a.ws_m : nullptr);
        put_state(a.ws_l + stx, 0.f, kCoherent ? a.ws_l : nullptr);
      }
    }
  }

  if constexpr (kMode == RangeMode::kArrive) {
    if (arrive_last(a.counters, (size_t)b * gridDim.x + blockIdx.x, (int)gridDim.z) && ph == 0)
      merge_heads4(a.ws_acc, a.ws_m, a.ws_l, a.merge_out, bh0, G, ns, lane);
  } else if constexpr (kMode == RangeMode::kMerge) {
    // Thread t < 64 G: head t / 64, dims 2 (t % 64) and 2 (t % 64) + 1. Wave w
    // staged splits [w ns / 4, (w + 1) ns / 4) in its slots 0, 1, ...
    __syncthreads();
    const int t = threadIdx.x;
    if (t < 64 * G) {
      const int h = t >> 6, d2 = t & 63;
      float M = kNegInf;
      for (int w = 0; w < kWavesPerHead; ++w) {
        const float* ml = lds + w * wave_floats + slots * G * kHeadDim;
        const int n = (w + 1) * ns / kWavesPerHead - w * ns / kWavesPerHead;
        for (int j = 0; j < n; ++j) M = fmaxf(M, ml[(j * G + h) * 2]);
      }
      float L = 0.f, A0 = 0.f, A1 = 0.f;
      for (int w = 0; w < kWavesPerHead; ++w) {
        const float* acc = lds + w * wave_floats;
        const float* ml = acc + slots * G * kHeadDim;
        const int n = (w + 1) * ns / kWavesPerHead - w * ns / kWavesPerHead;
        for (int j = 0; j < n; ++j) {
          const float2 m_l = *reinterpret_cast<const float2*>(ml + (j * G + h) * 2);
          const float2 x = reinterpret_cast<const float2*>(acc + (j * G + h) * kHeadDim)[d2];
          const float f = fold_factor(m_l.x, M);
          const bool first = w == 0 && j == 0;
          fold_term(first, m_l.y, f, L);
          fold_term(first, x.x, f, A0);
          fold_term(first, x.y, f, A1);
        }
      }
      reinterpret_cast<uint32_t*>(a.merge_out + (bh0 + h) * kHeadDim)[d2] =
          f32_to_bf16_bits(finalize(A0, L)) | (f32_to_bf16_bits(finalize(A1, L)) << 16);
    }
  }
}

// Log-sum-exp merge of the num_splits states of each (b, q-head) in split order
// (v2_splitkv.cu:92-108): one wave per (b, q-head) (merge_head), kBatch
// splits per memory round trip.
template <int kBatch>
__global__ __launch_bounds__(256) void gqa_decode_merge_kernel(const float* __restrict__ ws_acc,
                                                               const float* __restrict__ ws_m,
                                                               const float* __restrict__ ws_l,
                                                               uint16_t* __restrict__ out, int BH,
                                                               int ns) {
  const int bh = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (bh >= BH) return;
  merge_head<kBatch>(ws_acc, ws_m, ws_l, out, (size_t)bh, ns, threadIdx.x & 63);
}

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

// Workgroups per (request, kv-head, q-head chunk) of the split-range layout,
// or 0 for the shared-split layout. The single pass fills one round of one
// wave per SIMD with kWavesPerHead waves per pair when the batch is small
// enough; the split-range layout keeps that many waves per pair -- Z
// workgroups, Z = CUs / pairs, at least one -- and takes over once the splits
// are at least as many as those waves. Below that count the shared layout's
// num_splits x 4 waves per pair are at most one round, and it runs as before.
// Measured on MI355X (config 2, 32 requests x 8 kv-heads of 8192 tokens): the
// shared layout at 4 / 8 / 16 / 32 / 64 splits puts 4 / 8 / 16 / 32 / 64 waves
// on each SIMD, each with 32 / 16 / 8 / 4 / 2 tiles, and ran 176 / 179 / 191 /
// 211 / 243 us against 167 us for one split.
int split_range_groups(int B, int pairs_per_request, int num_splits) {
  if (num_splits < 2) return 0;
  const int cus = device_cu_count();
  const int64_t pairs = (int64_t)B * pairs_per_request;
  const int64_t z = cus > pairs ? cus / pairs : 1;
  return (int64_t)num_splits >= kWavesPerHead * z ? (int)z : 0;
}

// One split-range launch: grid (Hkv, B, z). merge: v2 with its merge folded
// in (one workgroup per pair, all of a wave's splits in its stage).
template <int G, bool kBlockUniform>
hipError_t launch_split_range(const ScanArgs& a, dim3 grid, bool merge, hipStream_t stream) {
  const int W = kWavesPerHead * (int)grid.z;
  const int slots = stage_slots(G, (a.num_splits + W - 1) / W);
  const size_t lds = (size_t)kWavesPerHead * stage_wave_floats(G, slots) * sizeof(float);
  const dim3 block(64 * kWavesPerHead);
  if (merge)
    hipLaunchKernelGGL((gqa_decode_split_range_kernel<G, kBlockUniform, RangeMode::kMerge>), grid,
                       block, lds, stream, a, slots);
  else if (a.counters)
    hipLaunchKernelGGL((gqa_decode_split_range_kernel<G, kBlockUniform, RangeMode::kArrive>),
                       grid, block, lds, stream, a, slots);
  else
    hipLaunchKernelGGL((gqa_decode_split_range_kernel<G, kBlockUniform, RangeMode::kStates>),
                       grid, block, lds, stream, a, slots);
  return hipGetLastError();
}

template <int G>
hipError_t launch_split_range_g(const ScanArgs& a, dim3 grid, bool merge, hipStream_t stream) {
  return a.block_size % kTile == 0 ? launch_split_range<G, true>(a, grid, merge, stream)
                                   : launch_split_range<G, false>(a, grid, merge, stream);
}

// Waves per split of the shared layout: kWavesPerHead, or 8, 12 or 16 where
// waves_per_split allows (max_p: 3 waves per SIMD for the 4-head scan's ~160
// VGPRs, 4 for the smaller ones; more would spill inside the tile loop). With
// few requests and splits (config 3 at 2 splits: 128 pairs x splits) the grid
// occupies only part of the CUs, and a workgroup can only use its own CU: the
// extra waves raise the rate at which each occupied CU streams its split.
// Full grids keep kWavesPerHead.
template <int GH>
hipError_t launch_scan_gh(const ScanArgs& a, int B, hipStream_t stream) {
  const dim3 grid(a.Hkv * a.nchunk, B, a.num_splits);
  constexpr int kMaxP = GH == 4 ? 12 : 16;
  switch (waves_per_split((int64_t)B * a.Hkv * a.nchunk, a.num_splits,
                          (int64_t)a.max_blocks * a.block_size, kWavesPerHead, kMaxP,
                          device_cu_count())) {
    case 16:
      if constexpr (kMaxP >= 16) return launch_scan_shape<GH, 16>(a, grid, stream);
      [[fallthrough]];
    case 12: return launch_scan_shape<GH, 12>(a, grid, stream);
    case 8: return launch_scan_shape<GH, 8>(a, grid, stream);
    default: return launch_scan_shape<GH, kWavesPerHead>(a, grid, stream);
  }
}

hipError_t launch_scan(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                       const int* block_table, const int* seq_lens, uint16_t* out, float* ws_acc,
                       float* ws_m, float* ws_l, int B, int Hq, int Hkv, int block_size,
                       int max_blocks, float scale, int num_splits, hipStream_t stream,
                       uint32_t* counters = nullptr, uint16_t* merge_out = nullptr,
                       bool* merged = nullptr) {
  // merge_out without counters: the caller (gqa_decode_v2_launch) would merge
  // the split states into merge_out with the merge kernel; a launch that
  // merges them itself sets *merged, and the caller then skips it.
  if (merged) *merged = false;
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
  a.counters = counters;
  a.merge_out = counters ? merge_out : nullptr;  // the single-launch mode's output
  if (use_mfma(a.G) || use_mfma_underfilled(B, a.Hkv, num_splits,
                                             (int64_t)max_blocks * block_size, device_cu_count()))
    return launch_scan_mfma(a, B, stream);
  // Groups of at most 4 q-heads (one chunk per kv-head, each wave serving the
  // whole group): the split-range layout where split_range_groups says so.
  // (Larger groups reach the VALU scan only in builds that move the
  // matrix-core threshold, and take the shared layout's head chunks.)
  const int z = a.G <= 4 ? split_range_groups(B, a.Hkv, num_splits) : 0;
  if (z > 0) {
    const dim3 grid(a.Hkv, B, z);
    // One workgroup per pair whose waves stage all their splits: the
    // workgroup merges them itself (the single-launch mode's counters are
    // then left untouched, at zero).
    const bool merge = merge_out != nullptr && z == 1 &&
                       (num_splits + kWavesPerHead - 1) / kWavesPerHead <= stage_cap(a.G);
    if (merge) {
      a.merge_out = merge_out;
      if (merged) *merged = true;
    }
    switch (a.G) {
      case 1: return launch_split_range_g<1>(a, grid, merge, stream);
      case 2: return launch_split_range_g<2>(a, grid, merge, stream);
      case 3: return launch_split_range_g<3>(a, grid, merge, stream);
      case 4: return launch_split_range_g<4>(a, grid, merge, stream);
      default: return hipErrorInvalidValue;
    }
  }
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
  // Round trips per head: ceil(ns / batch), each of batch acc rows per lane.
  const dim3 grid((BH + 3) / 4);
  if (num_splits <= 8)
    hipLaunchKernelGGL(gqa::gqa_decode_merge_kernel<8>, grid, dim3(256), 0, stream, ws_acc, ws_m,
                       ws_l, out, BH, num_splits);
  else if (num_splits <= 16)
    hipLaunchKernelGGL(gqa::gqa_decode_merge_kernel<16>, grid, dim3(256), 0, stream, ws_acc, ws_m,
                       ws_l, out, BH, num_splits);
  else if (num_splits <= 32)
    hipLaunchKernelGGL(gqa::gqa_decode_merge_kernel<32>, grid, dim3(256), 0, stream, ws_acc, ws_m,
                       ws_l, out, BH, num_splits);
  else
    hipLaunchKernelGGL(gqa::gqa_decode_merge_kernel<64>, grid, dim3(256), 0, stream, ws_acc, ws_m,
                       ws_l, out, BH, num_splits);
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
  hipError_t err = gqa::check_common(q, k_cache, v_cache, block_table, seq_lens, out, B, Hq, Hkv,
                                     block_size, max_blocks);
  if (err != hipSuccess) return err;
  if (num_splits < 1 || num_splits > GQA_DECODE_MAX_SPLITS) return hipErrorInvalidValue;
  if (B > 0 && (!ws_acc || !ws_m || !ws_l)) return hipErrorInvalidValue;
  if (B == 0) return hipSuccess;
  // The partial launch, which may merge into out itself (the split-range
  // layout with one workgroup per pair); else the merge launch.
  bool merged = false;
  err = gqa::launch_scan(q, k_cache, v_cache, block_table, seq_lens, nullptr, ws_acc, ws_m, ws_l,
                         B, Hq, Hkv, block_size, max_blocks, scale, num_splits, stream, nullptr,
                         out, &merged);
  if (err != hipSuccess || merged) return err;
  return gqa_decode_v2_merge_launch(ws_acc, ws_m, ws_l, out, B, Hq, num_splits, stream);
}

extern "C" size_t gqa_decode_v2_workspace_bytes(int B, int Hq, int num_splits) {
  if (B <= 0 || Hq <= 0 || num_splits <= 0) return 0;
  return (size_t)B * Hq * num_splits * (gqa::kHeadDim + 2) * sizeof(float);
}

namespace gqa {
namespace {

__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t* __restrict__ p, size_t n,
                                                       uint32_t v) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
    p[i] = v;
}

// The fused launch's workspace: one 32-bit arrival counter per (request,
// q-head) at its start -- enough for every launch layout's merge groups, a
// group holding at least one q-head -- and the v2 workspace (acc, m, l) at its
// end, starting at a 256-byte boundary. A workspace reset for the largest
// batch then serves any smaller one: the smaller launch's counters are a
// prefix of the zeroed ones, which every launch leaves zero, and its states
// stay clear of them.
struct FusedWorkspace {
  uint32_t* counters;
  float* acc;
  float* m;
  float* l;
};

size_t fused_counter_bytes(int B, int Hq) { return ((size_t)B * Hq * 4 + 255) & ~(size_t)255; }

hipError_t fused_workspace(void* workspace, size_t workspace_bytes, int B, int Hq, int num_splits,
                           FusedWorkspace& w) {
  if (num_splits < 1 || num_splits > GQA_DECODE_MAX_SPLITS) return hipErrorInvalidValue;
  if (!workspace || ((uintptr_t)workspace & 15) != 0) return hipErrorInvalidValue;
  if (workspace_bytes < gqa_decode_v2_fused_workspace_bytes(B, Hq, num_splits))
    return hipErrorInvalidValue;
  const size_t states = (size_t)B * Hq * num_splits;
  const size_t state_off = (workspace_bytes - states * (kHeadDim + 2) * 4) & ~(size_t)255;
  w.counters = static_cast<uint32_t*>(workspace);
  w.acc = reinterpret_cast<float*>(static_cast<char*>(workspace) + state_off);
  w.m = w.acc + states * kHeadDim;
  w.l = w.m + states;
  return hipSuccess;
}

}  // namespace
}  // namespace gqa

extern "C" size_t gqa_decode_v2_fused_workspace_bytes(int B, int Hq, int num_splits) {
  const size_t states = gqa_decode_v2_workspace_bytes(B, Hq, num_splits);
  return states ? gqa::fused_counter_bytes(B, Hq) + states : 0;
}

extern "C" int gqa_decode_v2_fused_reset(void* workspace, size_t workspace_bytes, int B, int Hq,
                                         int num_splits, hipStream_t stream) {
  if (B < 0 || Hq < 1 || (int64_t)B * Hq > (int64_t(1) << 30)) return hipErrorInvalidValue;
  if (B == 0) return hipSuccess;
  gqa::FusedWorkspace w;
  const hipError_t err = gqa::fused_workspace(workspace, workspace_bytes, B, Hq, num_splits, w);
  if (err != hipSuccess) return err;
  const size_t n = gqa::fused_counter_bytes(B, Hq) / 4;
  const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 1024);
  hipLaunchKernelGGL(gqa::fill_u32_kernel, dim3(blocks), dim3(256), 0, stream, w.counters, n, 0u);
  return hipGetLastError();
}

extern "C" int gqa_decode_v2_fused_launch(const uint16_t* q, const uint16_t* k_cache,
                                          const uint16_t* v_cache, const int* block_table,
                                          const int* seq_lens, uint16_t* out, int B, int Hq,
                                          int Hkv, int block_size, int max_blocks, float scale,
                                          int num_splits, void* workspace, size_t workspace_bytes,
                                          hipStream_t stream) {
  hipError_t err = gqa::check_common(q, k_cache, v_cache, block_table, seq_lens, out, B, Hq, Hkv,
                                     block_size, max_blocks);
  if (err != hipSuccess) return err;
  if (B == 0) return hipSuccess;
  gqa::FusedWorkspace w;
  err = gqa::fused_workspace(workspace, workspace_bytes, B, Hq, num_splits, w);
  if (err != hipSuccess) return err;
  if (num_splits == 1)  // the single-pass kernel, as gqa_decode_v2_launch runs it
    return gqa::launch_scan(q, k_cache, v_cache, block_table, seq_lens, out, w.acc, w.m, w.l, B,
                            Hq, Hkv, block_size, max_blocks, scale, 1, stream);
  return gqa::launch_scan(q, k_cache, v_cache, block_table, seq_lens, nullptr, w.acc, w.m, w.l, B,
                          Hq, Hkv, block_size, max_blocks, scale, num_splits, stream, w.counters,
                          out);
}

// Number of splits. For the matrix-core scan's slot-group layout (groups of
// 5-16 q-heads, 4 or 8 kv-heads; gqa_decode_mfma.hip): as many splits as give
// every CU one workgroup (8 waves), rounded down, no split longer than
// kSlotChunk tokens and none shorter than kSlotMinChunk -- when that grid does
// not give the layout its residency, the head-strided rule below applies.
// Measured on MI355X, 64Q/8KV: uniform B=32 S=32768 is fastest at 8 splits
// (637 us; 666 at 16), uniform B=64 S=8192 at 4 (329 us); ragged batches want
// more splits than the host can tell (B=32: 504 us at 8, 447 at 32; B=128
// with 16-token blocks: 1580 at 8, 1538 at 16). Splits of 1024 tokens still
// win (B=32 S=8192: 180 us at 8 vs 198 head-strided), splits of 256 lose
// (B=32 S=2048: 56 us at 8 vs 50 for one head-strided pass).
// Otherwise two bounds, the larger wins:
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
  if (num_cus <= 0 && (num_cus = gqa::device_cu_count()) <= 0) return 0;
  const int G = Hq / Hkv;
  const bool mfma = gqa::use_mfma(G);
  const int GH = mfma ? 16 : gqa::heads_per_wave(G);  // q-heads per wave
  const int P = gqa::kWavesPerHead;
  const int64_t s_max = (int64_t)max_blocks * block_size;
  if (mfma && gqa::mfma_slot_shape(Hkv, G)) {
    constexpr int64_t kSlotChunk = 4096;
    constexpr int64_t kSlotMinChunk = 1024;
    int64_t ns = (int64_t)8 * num_cus / ((int64_t)B * Hkv);
    const int64_t ns_len = (s_max + kSlotChunk - 1) / kSlotChunk;
    if (ns < ns_len) ns = ns_len;
    const int64_t ns_cap = s_max / kSlotMinChunk > 1 ? s_max / kSlotMinChunk : 1;
    if (ns > ns_cap) ns = ns_cap;
    if (ns > kMaxSplits) ns = kMaxSplits;
    if (ns < 1) ns = 1;
    if (gqa::use_mfma_slot(B, Hkv, G, (int)ns, num_cus)) return (int)ns;
  }
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
