// Token-balanced split-KV decode for gfx950: a persistent grid of one
// workgroup per CU, each taking an equal share of all the batch's tiles.
//
// The split-rule kernels give every request the same number of splits, so in
// a ragged batch the waves of long requests stream far longer than the rest,
// and the host cannot size the splits to the lengths without reading seq_lens
// back. Here the work is the concatenation, in (request, kv-head) order, of
// every segment's 16-token tiles: T = Hkv * sum_b ceil(S_b / 16) tiles.
// Workgroup w of nwg takes tiles [w*T/nwg, (w+1)*T/nwg) -- equal shares to
// within one tile, whatever the lengths -- and walks them segment by segment
// ("pieces"), scanning each piece with the VALU scan of gqa_scan_valu.hpp
// (P = 4 waves dealing the piece's tiles round-robin). A piece that is a whole
// segment is normalised and written to `out` directly; only the first and last
// piece of a workgroup can be partial, and their states go to two workspace
// slots. A second kernel merges each segment that was cut at a workgroup
// boundary, in workgroup order: results are bitwise reproducible for a given
// nwg.
//
// Each workgroup computes the tile prefix sums of the batch itself (from
// seq_lens, into LDS), so the host needs no lengths and launches a fixed grid.
// The LDS table is sized so that only one workgroup fits a CU: with nwg = the
// CU count that gives one wave per SIMD, the residency the split-rule kernels
// measured fastest. Lengths are clamped to max_blocks * block_size, so no
// block-table read leaves the request's row; a request of length 0 gets NaN,
// as 0/0 gives in the other kernels (and the reference).
//
// With 4 or 8 kv-heads (every group of up to 16 q-heads) the matrix-core
// variant below runs instead: a segment is a whole request (T = sum_b
// ceil(S_b / 16)), a workgroup holds one wave per kv-head, and every wave
// scans each piece of its share for its own kv-head with the MFMA scan of
// gqa_scan_mfma.hpp, so one CU reads each cache slot whole.
#include "gqa_device.hpp"
#include "gqa_launch.hpp"
#include "gqa_scan.hpp"
#include "gqa_scan_mfma.hpp"
#include "gqa_scan_valu.hpp"
#include "gqa_decode.h"

#include <mutex>
#include <type_traits>

namespace gqa {

// Requests the LDS prefix table holds. 20480 entries (80 KiB) also keep the
// LDS of one workgroup above half the CU's 160 KiB: one workgroup per CU.
constexpr int kBalancedTable = 20480;
constexpr int kBalancedMaxB = GQA_DECODE_BALANCED_MAX_BATCH;
static_assert(kBalancedMaxB < kBalancedTable, "prefix table holds B + 1 entries");
constexpr int kStateStride = 132;  // floats per slot state: acc[128], m, l, 2 pad (16-byte rows)

// What the merge kernel needs about the boundary at the end of share w,
// written by the share's workgroup: the batch's tile count and the segment
// its last piece belongs to, and whether that boundary cuts the segment and
// is the first boundary inside it (then the merge starts there).
struct ShareMeta {
  int T, seg0, seg1;  // all tiles; the segment's tile range
  int b, hkv, merge, pad0, pad1;
};

struct BalancedArgs {
  float* states;    // [nwg][2][GH][kStateStride]: first-piece and last-piece slots
  ShareMeta* meta;  // [nwg]
  int B, nwg, s_cap;
};

// Workspace layout: the state slots, then the share records (16-byte aligned).
inline size_t balanced_states_bytes(int nwg, int GH) {
  return ((size_t)nwg * 2 * GH * kStateStride * sizeof(float) + 15) & ~size_t(15);
}

// pre[b] = sum over requests b' < b of ceil(min(S_b', s_cap) / 16), for
// b = 0..B, computed by all NT threads of the workgroup in rounds of NT
// requests (coalesced loads, wave scans, a carry across rounds).
template <int NT>
__device__ __forceinline__ void tile_prefix(const int* __restrict__ seq_lens, int B, int s_cap,
                                            uint32_t* pre, uint32_t* wave_tot) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  constexpr int NW = NT / 64;
  uint32_t carry = 0;
  if (tid == 0) pre[0] = 0;
  for (int base = 0; base < B; base += NT) {
    const int b = base + tid;
    uint32_t x = 0;
    if (b < B) {
      const int s = min(max(seq_lens[b], 0), s_cap);
      x = (uint32_t)((s + kTile - 1) / kTile);
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    if (lane == 63) wave_tot[wv] = x;
    __syncthreads();
    uint32_t off = carry, total = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const uint32_t t = wave_tot[w];
      off += w < wv ? t : 0;
      total += t;
    }
    if (b < B) pre[b + 1] = off + x;
    carry += total;
    __syncthreads();  // wave_tot is rewritten next round; pre is complete after the last
  }
}

// The request whose tiles contain global tile t (0 <= t < T): the largest b
// with Hkv * pre[b] <= t. Requests without tiles are never returned. (The
// launcher guarantees every tile index, T included, fits in 31 bits.)
__device__ __forceinline__ int find_request(const uint32_t* pre, int B, int Hkv, int t) {
  int lo = 0, hi = B - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (Hkv * (int)pre[mid] <= t) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// Values every lane of the workgroup computed alike from LDS, made uniform
// for the compiler (scalar registers, scalar block-id loads in the scan).
__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ uint32_t uniform(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)x);
}

__device__ __forceinline__ int share_start(int w, int T, int nwg) {
  return (int)((int64_t)w * T / nwg);
}

__device__ __forceinline__ int clamped_len(const ScanArgs& a, int b, int s_cap) {
  return min(max(a.seq_lens[b], 0), s_cap);
}

template <int GH, int P, int DEPTH, bool kBlockUniform>
__global__ __launch_bounds__(64 * P) void gqa_decode_balanced_kernel(const ScanArgs a,
                                                                     const BalancedArgs ba) {
  __shared__ uint32_t pre[kBalancedTable];
  __shared__ uint32_t wave_tot[P];
  __shared__ WaveMergeLds<GH, P> lds;
  const int lane = threadIdx.x & 63;
  const int ph = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane >> 4, c = lane & 15;
  const int w = blockIdx.x;
  const int Hkv = a.Hkv, B = ba.B;

  tile_prefix<64 * P>(a.seq_lens, B, ba.s_cap, pre, wave_tot);
  const int T = Hkv * (int)uniform(pre[B]);
  const int t0 = share_start(w, T, ba.nwg), t1 = share_start(w + 1, T, ba.nwg);

  // Requests without tokens sit at position Hkv * pre[b] of the tile order;
  // the first workgroup whose share ends at or after it writes their NaN.
  for (int b = threadIdx.x; b < B; b += 64 * P) {
    const int p = Hkv * (int)pre[b];
    if (pre[b + 1] == pre[b] && t1 >= p && (w == 0 || t0 < p)) {
      uint32_t* o = reinterpret_cast<uint32_t*>(a.out + (size_t)b * a.Hq * kHeadDim);
      for (int i = 0; i < a.Hq * kHeadDim / 2; ++i) o[i] = 0x7fc07fc0u;  // bf16 quiet NaN pairs
    }
  }
  if (t0 >= t1) {
    if (threadIdx.x == 0) ba.meta[w] = ShareMeta{T, 0, 0, 0, 0, 0, 0, 0};
    return;
  }

  int b = uniform(find_request(pre, B, Hkv, t0));
  int req0 = Hkv * (int)uniform(pre[b]);
  int n = (int)uniform(pre[b + 1] - pre[b]);
  int hkv = (t0 - req0) / n;
  const int G = a.G;
  int t = t0;
  for (int piece = 0; t < t1; ++piece) {
    const int seg0 = req0 + hkv * n;
    const int lt0 = t - seg0;
    const int lt1 = min(t1, seg0 + n) - seg0;
    const int S = clamped_len(a, b, ba.s_cap);
    // The segment's kv-head: adjacent heads swapped, as in the split grid
    // (strided_kv_head), so a share whose segment index matches its
    // workgroup's XCD parity reads heads of the other parity (64Q/16KV, B=16,
    // S=8192: 172.0 -> 167.1 us).
    const int kvh = strided_kv_head(hkv, Hkv);
    const int h0 = kvh * G;

    uint4 qf[GH];
    load_q(a, b, h0, G, c, qf);
    WaveState<GH> st;
    init_state(st);
    scan_segment<GH, P, DEPTH, kBlockUniform, true>(a, a.block_table + (size_t)b * a.max_blocks,
                                                    kvh, qf, kTile * lt0, min(S, kTile * lt1), ph,
                                                    r, c, st);
    float Mw[GH], Lw[GH];
    merge_rows(st, Mw, Lw);
    __syncthreads();  // the previous piece's reads of lds are done
    stage_wave_state(lds, ph, lane, r, c, st, Mw, Lw);
    __syncthreads();

    const bool whole = lt0 == 0 && lt1 == n;
    // Only a workgroup's first and last pieces can be partial: slot 0 / 1.
    float* slot = ba.states + ((size_t)w * 2 + (piece == 0 ? 0 : 1)) * GH * kStateStride;
    for (int idx = threadIdx.x; idx < G * kHeadDim; idx += 64 * P) {
      const int h = idx / kHeadDim, d = idx % kHeadDim;
      float M, L, A;
      merge_wave_states(lds, h, d, M, L, A);
      if (whole) {
        a.out[((size_t)b * a.Hq + h0 + h) * kHeadDim + d] = (uint16_t)f32_to_bf16_bits(finalize(A, L));
      } else {
        float* sh = slot + h * kStateStride;
        sh[d] = A;
        if (d == 0) {
          sh[kHeadDim] = M;  // base-2 units
          sh[kHeadDim + 1] = L;
        }
      }
    }

    // The share's record, at its last piece: the boundary after it cuts the
    // segment if the piece ends early, and is the segment's first cut (where
    // the merge starts) if the piece also starts at the segment's start.
    if (threadIdx.x == 0 && seg0 + lt1 >= t1)
      ba.meta[w] = ShareMeta{T, seg0, seg0 + n, b, kvh, lt0 == 0 && lt1 < n, 0, 0};
    t = seg0 + lt1;
    if (++hkv == Hkv) {
      hkv = 0;
      do {
        ++b;
      } while (b < B && uniform(pre[b + 1]) == uniform(pre[b]));
      if (b < B) {
        req0 = Hkv * (int)uniform(pre[b]);
        n = (int)uniform(pre[b + 1] - pre[b]);
      }
    }
  }
}

// Workgroup w merges the segment whose first cut is the boundary after share
// w (the share's record says so; otherwise it exits at once). The segment's
// pieces are in shares w .. vend - 1: the first one's in its last-piece slot
// unless the segment is that share's first piece, every later one's in its
// first-piece slot. Wave i folds pieces i, i + P, ... in order with an online
// merge (lane l owns dims 2l, 2l + 1 of every head), loading a batch of pieces
// before folding it; the P wave results are then combined in wave order:
// bitwise reproducible.
template <int GH, int P>
__global__ __launch_bounds__(64 * P) void gqa_decode_balanced_merge_kernel(const ScanArgs a,
                                                                           const BalancedArgs ba) {
  constexpr int kBatch = 4;  // pieces a wave loads together
  __shared__ WaveMergeLds<GH, P> lds;
  const int w = blockIdx.x;
  const ShareMeta meta = ba.meta[w];
  if (!meta.merge) return;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwg = ba.nwg, G = a.G;
  const int T = meta.T, seg0 = meta.seg0, seg1 = meta.seg1;
  // Shares starting before seg1: share_start(v) < seg1 <=> v * T < seg1 * nwg.
  const int vend = (int)min((int64_t)nwg, ((int64_t)seg1 * nwg + T - 1) / T);

  float M[GH], L[GH];
  float2 A[GH];
#pragma unroll
  for (int h = 0; h < GH; ++h) {
    M[h] = kNegInf;
    L[h] = 0.f;
    A[h] = make_float2(0.f, 0.f);
  }
  for (int v = w + wv; v < vend; v += kBatch * P) {
    float mv[kBatch][GH], lv[kBatch][GH];
    float2 av[kBatch][GH];
    bool live[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int u = v + k * P;
      const int u0 = share_start(u, T, nwg), u1 = share_start(u + 1, T, nwg);
      live[k] = u < vend && u1 > u0;  // an empty share holds no piece
      const float* base = ba.states + ((size_t)(live[k] ? u : w) * 2 + (u0 < seg0 ? 1 : 0)) *
                                          GH * kStateStride;
#pragma unroll
      for (int h = 0; h < GH; ++h) {
        const float* sh = base + (h < G ? h : 0) * kStateStride;
        mv[k][h] = sh[kHeadDim];
        lv[k][h] = sh[kHeadDim + 1];
        av[k][h] = reinterpret_cast<const float2*>(sh)[lane];
      }
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      if (!live[k]) continue;
#pragma unroll
      for (int h = 0; h < GH; ++h) {
        const float mn = fmaxf(M[h], mv[k][h]);
        const float ms = mn == kNegInf ? 0.f : mn;
        const float fa = exp2_fast(M[h] - ms), fv = exp2_fast(mv[k][h] - ms);
        L[h] = fmaf(L[h], fa, lv[k][h] * fv);
        A[h].x = fmaf(A[h].x, fa, av[k][h].x * fv);
        A[h].y = fmaf(A[h].y, fa, av[k][h].y * fv);
        M[h] = mn;
      }
    }
  }
#pragma unroll
  for (int h = 0; h < GH; ++h) {
    reinterpret_cast<float2*>(&lds.acc[wv][h][0])[lane] = A[h];
    if (lane == 0) {
      lds.m[wv][h] = M[h];
      lds.l[wv][h] = L[h];
    }
  }
  __syncthreads();
  const int h0 = meta.hkv * G;
  for (int idx = threadIdx.x; idx < G * kHeadDim; idx += 64 * P) {
    const int h = idx / kHeadDim, d = idx % kHeadDim;
    float Mh, Lh, Ah;
    merge_wave_states(lds, h, d, Mh, Lh, Ah);
    a.out[((size_t)meta.b * a.Hq + h0 + h) * kHeadDim + d] =
        (uint16_t)f32_to_bf16_bits(finalize(Ah, Lh));
  }
}

template <int GH>
hipError_t launch_balanced_partial(const ScanArgs& a, const BalancedArgs& ba, hipStream_t stream) {
  constexpr int P = kWavesPerHead;
  if (a.block_size % kTile == 0)
    hipLaunchKernelGGL((gqa_decode_balanced_kernel<GH, P, kScanDepth, true>), dim3(ba.nwg),
                       dim3(64 * P), 0, stream, a, ba);
  else
    hipLaunchKernelGGL((gqa_decode_balanced_kernel<GH, P, kScanDepth, false>), dim3(ba.nwg),
                       dim3(64 * P), 0, stream, a, ba);
  return hipGetLastError();
}

template <int GH>
hipError_t launch_balanced_merge(const ScanArgs& a, const BalancedArgs& ba, hipStream_t stream) {
  constexpr int P = kWavesPerHead;
  if (ba.nwg < 2) return hipSuccess;  // one share: every piece was whole
  hipLaunchKernelGGL((gqa_decode_balanced_merge_kernel<GH, P>), dim3(ba.nwg - 1), dim3(64 * P), 0,
                     stream, a, ba);
  return hipGetLastError();
}


// ---------------------------------------------------------------------------
// The same token-balanced split-KV on the matrix-core scan in its slot-group
// layout, for every group of up to 16 q-heads over 4 or 8 kv-heads: a
// workgroup holds one wave per kv-head, a segment is a whole request
// (T = sum_b ceil(S_b / 16) tiles), and every wave scans each piece of its
// share for its own kv-head, so the waves of a CU read each cache slot whole
// at about the same time (see gqa_decode_mfma.hip). A piece that is a whole request is
// normalised and written to `out`; a workgroup's first and last pieces go to
// its two state slots, each holding all Hq q-heads.
template <int NW, bool kBlockUniform>
__global__ __launch_bounds__(64 * NW) void gqa_decode_balanced_mfma_kernel(const ScanArgs a,
                                                                           const BalancedArgs ba) {
  static_assert(kMTile == kTile, "the tile prefix sums count 16-token tiles");
  __shared__ uint32_t pre[kBalancedTable];
  __shared__ uint32_t wave_tot[NW];
  __shared__ __attribute__((aligned(16))) uint8_t vlds_all[NW][kMTile * 256];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // the wave's kv-head
  const int j = lane & 15, g = lane >> 4;
  const int w = blockIdx.x;
  const int B = ba.B, G = a.G, Hq = a.Hq;

  tile_prefix<64 * NW>(a.seq_lens, B, ba.s_cap, pre, wave_tot);
  const int T = (int)uniform(pre[B]);
  const int t0 = share_start(w, T, ba.nwg), t1 = share_start(w + 1, T, ba.nwg);

  // Requests without tokens sit at position pre[b] of the tile order; the
  // first workgroup whose share ends at or after it writes their NaN.
  for (int b = threadIdx.x; b < B; b += 64 * NW) {
    const int p = (int)pre[b];
    if (pre[b + 1] == pre[b] && t1 >= p && (w == 0 || t0 < p)) {
      uint32_t* o = reinterpret_cast<uint32_t*>(a.out + (size_t)b * Hq * kHeadDim);
      for (int i = 0; i < Hq * kHeadDim / 2; ++i) o[i] = 0x7fc07fc0u;  // bf16 quiet NaN pairs
    }
  }
  if (t0 >= t1) {
    if (threadIdx.x == 0) ba.meta[w] = ShareMeta{T, 0, 0, 0, 0, 0, 0, 0};
    return;
  }

  int b = uniform(find_request(pre, B, 1, t0));
  const int h0 = wv * G;  // the wave's q-heads: h0 .. h0 + G - 1
  int t = t0;
  for (int piece = 0; t < t1; ++piece) {
    const int seg0 = (int)uniform(pre[b]);
    const int n = (int)uniform(pre[b + 1]) - seg0;
    const int lt0 = t - seg0;
    const int lt1 = min(t1, seg0 + n) - seg0;
    const int S = clamped_len(a, b, ba.s_cap);

    uint4 qf[4];
    mfma_load_q(a, b, h0, G, j, g, qf);
    MfmaState st;
    mfma_init(st);
    mfma_scan_segment<kMTile, kBlockUniform>(a, a.block_table + (size_t)b * a.max_blocks, wv, qf,
                                             kMTile * lt0, min(S, kMTile * lt1), 0, 1,
                                             vlds_all[wv], j, g, st);
    float Me[4], Le[4];
    mfma_finish(st, g, Me, Le);

    const bool whole = lt0 == 0 && lt1 == n;
    // Only a workgroup's first and last pieces can be partial: slot 0 / 1.
    float* slot = ba.states + ((size_t)w * 2 + (piece == 0 ? 0 : 1)) * Hq * kStateStride;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int h = 4 * g + e;
      if (h >= G) continue;
      if (whole) {
        uint16_t* o = a.out + ((size_t)b * Hq + h0 + h) * kHeadDim;
#pragma unroll
        for (int nb = 0; nb < 8; ++nb)
          o[16 * nb + j] = (uint16_t)f32_to_bf16_bits(finalize(st.o[nb][e], Le[e]));
      } else {
        float* sh = slot + (h0 + h) * kStateStride;
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) sh[16 * nb + j] = st.o[nb][e];
        if (j == 0) {
          sh[kHeadDim] = Me[e];  // base-2 units
          sh[kHeadDim + 1] = Le[e];
        }
      }
    }

    // The share's record, at its last piece (as in the VALU kernel above).
    if (threadIdx.x == 0 && seg0 + lt1 >= t1)
      ba.meta[w] = ShareMeta{T, seg0, seg0 + n, b, 0, lt0 == 0 && lt1 < n, 0, 0};
    t = seg0 + lt1;
    do {
      ++b;
    } while (b < B && uniform(pre[b + 1]) == uniform(pre[b]));
  }
}

// Workgroup (w, y) merges q-heads y * NWM .. y * NWM + NWM - 1 of the request
// whose first cut is the boundary after share w (its record says so;
// otherwise it exits at once). The request's pieces are in shares
// w .. vend - 1, found as in the VALU merge. Each wave folds one head's pieces
// in share order with an online merge (lane l owns dims 2l, 2l + 1), loading
// kBatch pieces at a time: bitwise reproducible for a given number of
// workgroups. One wave per head keeps the merge to one or two memory round
// trips (a workgroup walking the heads in turn took ~30 us on config 4).
template <int NWM>
__global__ __launch_bounds__(64 * NWM) void gqa_decode_balanced_mfma_merge_kernel(
    const ScanArgs a, const BalancedArgs ba) {
  constexpr int kBatch = 8;  // pieces a wave loads together
  const int w = blockIdx.x;
  const ShareMeta meta = ba.meta[w];
  if (!meta.merge) return;
  const int lane = threadIdx.x & 63;
  const int h = blockIdx.y * NWM + (threadIdx.x >> 6);
  const int nwg = ba.nwg, Hq = a.Hq;
  if (h >= Hq) return;
  const int T = meta.T, seg0 = meta.seg0, seg1 = meta.seg1;
  const int vend = (int)min((int64_t)nwg, ((int64_t)seg1 * nwg + T - 1) / T);
  float M = kNegInf, L = 0.f;
  float2 A = make_float2(0.f, 0.f);
  for (int v = w; v < vend; v += kBatch) {
    float mv[kBatch], lv[kBatch];
    float2 av[kBatch];
    bool live[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int u = v + k;
      const int u0 = share_start(u, T, nwg), u1 = share_start(u + 1, T, nwg);
      live[k] = u < vend && u1 > u0;  // an empty share holds no piece
      const float* sh = ba.states +
                        ((size_t)(live[k] ? u : w) * 2 + (u0 < seg0 ? 1 : 0)) * Hq * kStateStride +
                        (size_t)h * kStateStride;
      mv[k] = sh[kHeadDim];
      lv[k] = sh[kHeadDim + 1];
      av[k] = reinterpret_cast<const float2*>(sh)[lane];
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      if (!live[k]) continue;
      const float mn = fmaxf(M, mv[k]);
      const float ms = mn == kNegInf ? 0.f : mn;
      const float fa = exp2_fast(M - ms), fv = exp2_fast(mv[k] - ms);
      L = fmaf(L, fa, lv[k] * fv);
      A.x = fmaf(A.x, fa, av[k].x * fv);
      A.y = fmaf(A.y, fa, av[k].y * fv);
      M = mn;
    }
  }
  const uint32_t lo = f32_to_bf16_bits(finalize(A.x, L));
  const uint32_t hi = f32_to_bf16_bits(finalize(A.y, L));
  reinterpret_cast<uint32_t*>(a.out + ((size_t)meta.b * Hq + h) * kHeadDim)[lane] =
      lo | (hi << 16);
}

template <int NW>
hipError_t launch_balanced_mfma_partial(const ScanArgs& a, const BalancedArgs& ba,
                                        hipStream_t stream) {
  if (a.block_size % kMTile == 0)
    hipLaunchKernelGGL((gqa_decode_balanced_mfma_kernel<NW, true>), dim3(ba.nwg), dim3(64 * NW),
                       0, stream, a, ba);
  else
    hipLaunchKernelGGL((gqa_decode_balanced_mfma_kernel<NW, false>), dim3(ba.nwg), dim3(64 * NW),
                       0, stream, a, ba);
  return hipGetLastError();
}

hipError_t launch_balanced_mfma_merge(const ScanArgs& a, const BalancedArgs& ba,
                                      hipStream_t stream) {
  if (ba.nwg < 2) return hipSuccess;  // one share: every piece was whole
  hipLaunchKernelGGL((gqa_decode_balanced_mfma_merge_kernel<4>),
                     dim3(ba.nwg - 1, (a.Hq + 3) / 4), dim3(256), 0, stream, a, ba);
  return hipGetLastError();
}

// Groups of at least this many q-heads over 4 or 8 kv-heads take the
// matrix-core balanced scan: every such group by default. A profiling build
// with 5 (build.py --variant ... --define GQA_BALANCED_MFMA_MIN_GROUP=5)
// keeps groups of up to 4 on the VALU balanced scan, the other side of the
// measurement behind this default.
#ifndef GQA_BALANCED_MFMA_MIN_GROUP
#define GQA_BALANCED_MFMA_MIN_GROUP 1
#endif
inline bool balanced_mfma(int Hkv, int G) {
  return mfma_slot_shape(Hkv, G) && G >= GQA_BALANCED_MFMA_MIN_GROUP;
}

int balanced_workgroups(int num_workgroups) {
  return num_workgroups > 0 ? num_workgroups : device_cu_count();
}

}  // namespace gqa

extern "C" size_t gqa_decode_balanced_workspace_bytes(int B, int Hq, int Hkv, int num_workgroups) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0) return 0;
  const int G = Hq / Hkv;
  if (G > GQA_DECODE_BALANCED_MAX_GROUP) return 0;
  if (gqa::use_mfma(G) && !gqa::mfma_slot_shape(Hkv, G)) return 0;
  const int nwg = gqa::balanced_workgroups(num_workgroups);
  if (nwg <= 0) return 0;
  // State slots hold one kv-head's q-heads (VALU scan) or all Hq (MFMA scan).
  const int slot_heads = gqa::balanced_mfma(Hkv, G) ? Hq : gqa::heads_per_wave(G);
  return gqa::balanced_states_bytes(nwg, slot_heads) + (size_t)nwg * sizeof(gqa::ShareMeta);
}

namespace {

enum class BalancedPart { kBoth, kPartial, kMerge };

// Checks, argument packing and launch of one or both balanced kernels.
int balanced_launch(BalancedPart part, const uint16_t* q, const uint16_t* k_cache,
                    const uint16_t* v_cache, const int* block_table, const int* seq_lens,
                    uint16_t* out, int B, int Hq, int Hkv, int block_size, int max_blocks,
                    float scale, int num_workgroups, float* workspace, size_t workspace_bytes,
                    hipStream_t stream) {
  hipError_t err = gqa::check_common(q, k_cache, v_cache, block_table, seq_lens, out, B, Hq, Hkv,
                                     block_size, max_blocks);
  if (err != hipSuccess) return err;
  if (B == 0) return hipSuccess;
  const int G = Hq / Hkv;
  if (G > GQA_DECODE_BALANCED_MAX_GROUP || B > gqa::kBalancedMaxB) return hipErrorInvalidValue;
  // The matrix-core scan wherever its slot-group layout fits (4 or 8
  // kv-heads), also for groups of up to 4 q-heads: measured on MI355X it
  // streams 4-11 % faster than the VALU scan's (request, kv-head) shares on
  // ragged and uniform batches alike (config 5: 1185 vs 1229 us; ragged B=64,
  // 32768 tokens, groups of 1/2/3: 642/644/646 vs 684/688/709 us). Other
  // kv-head counts keep the VALU scan (groups of up to 4).
  const bool mfma = gqa::balanced_mfma(Hkv, G);
  if (gqa::use_mfma(G) && !mfma) return hipErrorInvalidValue;
  const int64_t s_cap = (int64_t)max_blocks * block_size;
  // Every tile index of the batch, segs * sum_b ceil(S_b / 16), fits in 31 bits
  // (Hkv segments per request for the VALU scan, one for the MFMA scan).
  const int64_t segs = mfma ? 1 : Hkv;
  if (segs * B * ((s_cap + gqa::kTile - 1) / gqa::kTile) >= (int64_t(1) << 31))
    return hipErrorInvalidValue;
  const int nwg = gqa::balanced_workgroups(num_workgroups);
  if (nwg <= 0) return hipErrorInvalidValue;
  if (!workspace || workspace_bytes < gqa_decode_balanced_workspace_bytes(B, Hq, Hkv, nwg))
    return hipErrorInvalidValue;

  gqa::ScanArgs a{};
  a.q = q;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.block_table = block_table;
  a.seq_lens = seq_lens;
  a.out = out;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.G = G;
  a.nchunk = 1;
  a.block_size = block_size;
  a.max_blocks = max_blocks;
  a.num_splits = 1;
  a.bs_div = gqa::make_fastdiv((uint32_t)block_size);
  a.scale_log2e = (float)((double)scale * 1.4426950408889634);
  const size_t states =
      gqa::balanced_states_bytes(nwg, mfma ? Hq : gqa::heads_per_wave(G));
  const gqa::BalancedArgs ba{workspace,
                             reinterpret_cast<gqa::ShareMeta*>(
                                 reinterpret_cast<char*>(workspace) + states),
                             B, nwg, (int)s_cap};
  if (mfma) {
    if (part != BalancedPart::kMerge) {
      const hipError_t e = Hkv == 4 ? gqa::launch_balanced_mfma_partial<4>(a, ba, stream)
                                    : gqa::launch_balanced_mfma_partial<8>(a, ba, stream);
      if (e != hipSuccess || part == BalancedPart::kPartial) return e;
    }
    return gqa::launch_balanced_mfma_merge(a, ba, stream);
  }
  auto run = [&](auto gh) -> int {
    constexpr int GH = decltype(gh)::value;
    if (part != BalancedPart::kMerge) {
      const hipError_t e = gqa::launch_balanced_partial<GH>(a, ba, stream);
      if (e != hipSuccess || part == BalancedPart::kPartial) return e;
    }
    return gqa::launch_balanced_merge<GH>(a, ba, stream);
  };
  switch (gqa::heads_per_wave(G)) {
    case 1: return run(std::integral_constant<int, 1>{});
    case 2: return run(std::integral_constant<int, 2>{});
    default: return run(std::integral_constant<int, 4>{});
  }
}

}  // namespace

extern "C" int gqa_decode_balanced_launch(const uint16_t* q, const uint16_t* k_cache,
                                          const uint16_t* v_cache, const int* block_table,
                                          const int* seq_lens, uint16_t* out, int B, int Hq,
                                          int Hkv, int block_size, int max_blocks, float scale,
                                          int num_workgroups, float* workspace,
                                          size_t workspace_bytes, hipStream_t stream) {
  return balanced_launch(BalancedPart::kBoth, q, k_cache, v_cache, block_table, seq_lens, out, B,
                         Hq, Hkv, block_size, max_blocks, scale, num_workgroups, workspace,
                         workspace_bytes, stream);
}

extern "C" int gqa_decode_balanced_partial_launch(
    const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, const int* block_table,
    const int* seq_lens, uint16_t* out, int B, int Hq, int Hkv, int block_size, int max_blocks,
    float scale, int num_workgroups, float* workspace, size_t workspace_bytes,
    hipStream_t stream) {
  return balanced_launch(BalancedPart::kPartial, q, k_cache, v_cache, block_table, seq_lens, out,
                         B, Hq, Hkv, block_size, max_blocks, scale, num_workgroups, workspace,
                         workspace_bytes, stream);
}

extern "C" int gqa_decode_balanced_merge_launch(
    const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, const int* block_table,
    const int* seq_lens, uint16_t* out, int B, int Hq, int Hkv, int block_size, int max_blocks,
    float scale, int num_workgroups, float* workspace, size_t workspace_bytes,
    hipStream_t stream) {
  return balanced_launch(BalancedPart::kMerge, q, k_cache, v_cache, block_table, seq_lens, out, B,
                         Hq, Hkv, block_size, max_blocks, scale, num_workgroups, workspace,
                         workspace_bytes, stream);
}

// The allocation-free launch's workspace: a file-scope device array, one copy
// per device at that device's own address. In host code `scratch` names a
// host-side stand-in, never the device memory: kernels get the address that
// hipGetSymbolAddress returns for the device, looked up once per device with
// that device current and kept here.
static __device__ __align__(256) uint8_t scratch[GQA_DECODE_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The device `stream` belongs to (the current device for the null stream).
hipError_t stream_device(hipStream_t stream, int* dev) {
  hipError_t err = hipGetDevice(dev);
  if (err == hipSuccess && stream != nullptr) err = hipStreamGetDevice(stream, dev);
  if (err == hipSuccess && (*dev < 0 || *dev >= kMaxDevices)) err = hipErrorInvalidDevice;
  return err;
}

// Device address of `scratch` on device dev, looked up on the first call for
// that device (with dev current) and kept. The lookup may load the library's
// code object on that device, which a stream being captured into a graph must
// not see: a first call while `stream` is capturing is refused.
hipError_t scratch_for_device(int dev, hipStream_t stream, void** ptr) {
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    hipError_t err = hipStreamIsCapturing(stream, &capture);
    if (err != hipSuccess) return err;
    if (capture != hipStreamCaptureStatusNone) return hipErrorStreamCaptureUnsupported;
    int cur = 0;
    if ((err = hipGetDevice(&cur)) != hipSuccess) return err;
    if (dev != cur && (err = hipSetDevice(dev)) != hipSuccess) return err;
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) {
      const hipError_t back = hipSetDevice(cur);
      if (err == hipSuccess) err = back;
    }
    if (err != hipSuccess) return err;
    if (p == nullptr || ((uintptr_t)p & 255) != 0) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return hipSuccess;
}

}  // namespace

extern "C" int gqa_decode_balanced_launch_noalloc(
    const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, const int* block_table,
    const int* seq_lens, uint16_t* out, int B, int Hq, int Hkv, int block_size, int max_blocks,
    float scale, int num_workgroups, hipStream_t stream) {
  // Scratch, workspace size and default workgroup count all come from the
  // device the stream belongs to.
  int dev = 0;
  hipError_t err = stream_device(stream, &dev);
  if (err != hipSuccess) return err;
  if (num_workgroups <= 0) {
    err = hipDeviceGetAttribute(&num_workgroups, hipDeviceAttributeMultiprocessorCount, dev);
    if (err != hipSuccess) return err;
  }
  const size_t need = gqa_decode_balanced_workspace_bytes(B, Hq, Hkv, num_workgroups);
  if (need == 0)  // B == 0 (nothing to do) or arguments the launcher rejects
    return balanced_launch(BalancedPart::kBoth, q, k_cache, v_cache, block_table, seq_lens, out,
                           B, Hq, Hkv, block_size, max_blocks, scale, num_workgroups, nullptr, 0,
                           stream);
  if (need > GQA_DECODE_NOALLOC_SCRATCH_BYTES) return hipErrorOutOfMemory;
  void* ws = nullptr;
  if ((err = scratch_for_device(dev, stream, &ws)) != hipSuccess) return err;
  return balanced_launch(BalancedPart::kBoth, q, k_cache, v_cache, block_table, seq_lens, out, B,
                         Hq, Hkv, block_size, max_blocks, scale, num_workgroups,
                         static_cast<float*>(ws), GQA_DECODE_NOALLOC_SCRATCH_BYTES, stream);
}

extern "C" int gqa_decode_prefer_balanced(int B, int Hq, int Hkv, int block_size, int max_blocks,
                                          int num_cus) {
  // Measured on MI355X over the 64-cell matrix and ragged batches: the
  // token-balanced launch wins where the split-rule grid is uneven -- ragged
  // lengths, or more waves than one per SIMD (a grid the split heuristic could
  // not make exactly one round) -- and where many splits make the split merge
  // heavy, as long as segments are long enough that restarting the load
  // pipeline at each piece stays cheap. It loses a few percent where the split
  // grid is exactly one round of one wave per SIMD with few splits (uniform
  // lengths make that perfect) and on short or small batches.
  // Groups of at most 4 q-heads: preferred when sequences reach at least
  // kMinLongest tokens, at least kMinBytes of KV, at most kMaxSegmentsPerCu
  // segments per CU, and a split grid that is not exactly one round of at
  // most kMaxEvenSplits splits.
  // Groups of 5-16 q-heads over 4 or 8 kv-heads (the matrix-core scan): the
  // balanced launch is within 1.5 % of the best split count on uniform
  // batches of at least kMfmaMinBatch requests and kMfmaMinBytes of KV
  // (64Q/8KV: B=32 S=32768 640 vs 637 us; B=64 S=8192 333 vs 329; B=16 S=8192
  // 95.0 vs 95.5) and far ahead on ragged ones (B=32: 344 vs 447; B=128: 1201
  // vs 1536; B=8: 100 vs 140); with fewer requests each is cut into many
  // pieces and the merge costs more (B=1 S=32768: 81 vs 36 us; B=8 S=8192: 59
  // vs 51), so below either bound the split launch runs.
  // Groups of at most 4 over 4 or 8 kv-heads run the matrix-core scan too, on
  // whole requests, so they take the same batch bound on top of their own rule:
  // one request cut into a piece per CU loses (32Q/8KV B=1: S=8192 67.5 vs
  // 21.0 us, S=32768 81.7 vs 34.8), while at B >= 32 with long sequences the
  // balanced launch wins by 3-6 % (B=128 S=8192: 641 vs 667 us).
  constexpr int64_t kMinLongest = 6144;
  constexpr int64_t kMinBytes = int64_t(32) << 20;
  constexpr int kMaxSegmentsPerCu = 16;
  constexpr int kMaxEvenSplits = 8;
  constexpr int kMfmaMinBatch = 8;
  constexpr int64_t kMfmaMinBytes = int64_t(512) << 20;
  if (num_cus <= 0 && (num_cus = gqa::device_cu_count()) <= 0) return 0;
  if (B < 1 || Hkv < 1 || Hq % Hkv != 0 || Hq / Hkv > GQA_DECODE_BALANCED_MAX_GROUP ||
      B > gqa::kBalancedMaxB || block_size < 1 || max_blocks < 1)
    return 0;
  const int G = Hq / Hkv;
  const int64_t s_cap = (int64_t)max_blocks * block_size;
  const int64_t kv_bytes = (int64_t)B * s_cap * Hkv * gqa::kHeadDim * 4;
  if (gqa::use_mfma(G)) {
    if (!gqa::mfma_slot_shape(Hkv, G)) return 0;
    if ((int64_t)B * ((s_cap + gqa::kTile - 1) / gqa::kTile) >= (int64_t(1) << 31)) return 0;
    return B >= kMfmaMinBatch && kv_bytes >= kMfmaMinBytes ? 1 : 0;
  }
  if ((int64_t)Hkv * B * ((s_cap + gqa::kTile - 1) / gqa::kTile) >= (int64_t(1) << 31)) return 0;
  if (gqa::balanced_mfma(Hkv, G) && B < kMfmaMinBatch) return 0;
  if (s_cap < kMinLongest || kv_bytes < kMinBytes) return 0;
  if ((int64_t)B * Hkv > (int64_t)kMaxSegmentsPerCu * num_cus) return 0;
  const int ns = gqa_decode_pick_num_splits(B, Hq, Hkv, block_size, max_blocks, num_cus);
  const int64_t split_waves = (int64_t)B * Hkv * gqa::kWavesPerHead * ns;
  return split_waves == (int64_t)num_cus * 4 && ns <= kMaxEvenSplits ? 0 : 1;
}
