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
#include "gqa_device.hpp"
#include "gqa_launch.hpp"
#include "gqa_merge.hpp"
#include "gqa_scan.hpp"
#include "gqa_scan_valu.hpp"
#include "gqa_decode.h"

#include <algorithm>

namespace gqa {

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
        if (a.ws_acc) {
          const size_t stx = bh * ns + split;
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
            put_state(a.ws_m + stx, Mw[h] * kLn2, a.counters);  // back to natural-log units
            put_state(a.ws_l + stx, Lw[h], a.counters);
          }
        }
      }
    }
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

// Log-sum-exp merge of the num_splits states of each (b, q-head) in split order
// (v2_splitkv.cu:92-108): one wave per (b, q-head) (merge_head).
__global__ __launch_bounds__(256) void gqa_decode_merge_kernel(const float* __restrict__ ws_acc,
                                                               const float* __restrict__ ws_m,
                                                               const float* __restrict__ ws_l,
                                                               uint16_t* __restrict__ out, int BH,
                                                               int ns) {
  const int bh = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (bh >= BH) return;
  merge_head(ws_acc, ws_m, ws_l, out, (size_t)bh, ns, threadIdx.x & 63);
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

template <int GH>
hipError_t launch_scan_gh(const ScanArgs& a, int B, hipStream_t stream) {
  const dim3 grid(a.Hkv * a.nchunk, B, a.num_splits);
  return launch_scan_shape<GH, kWavesPerHead>(a, grid, stream);
}

hipError_t launch_scan(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                       const int* block_table, const int* seq_lens, uint16_t* out, float* ws_acc,
                       float* ws_m, float* ws_l, int B, int Hq, int Hkv, int block_size,
                       int max_blocks, float scale, int num_splits, hipStream_t stream,
                       uint32_t* counters = nullptr, uint16_t* merge_out = nullptr) {
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
  a.merge_out = merge_out;
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
