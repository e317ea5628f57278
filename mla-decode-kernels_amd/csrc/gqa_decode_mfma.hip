// Single-pass / split-KV partial scan on the gfx950 matrix cores, used for
// GQA groups of 5 or more q-heads (16 per MFMA column block, larger groups in
// chunks of 16), and for smaller groups on grids that leave CUs idle with
// splits of at most 1024 tokens (use_mfma_underfilled in gqa_scan.hpp): the
// per-tile work is the MFMA scan of gqa_scan_mfma.hpp; this file holds the
// split-rule kernel and its launches.
//
// Same split rule, workspace contract and fixed-order merges as the VALU scan
// in gqa_decode_split.hip, including the single-launch mode.
#include "gqa_device.hpp"
#include "gqa_launch.hpp"
#include "gqa_merge.hpp"
#include "gqa_scan.hpp"
#include "gqa_scan_mfma.hpp"

namespace gqa {

namespace {

constexpr int kMWavesPerHead = 4;

// Two launch layouts. Head-strided (kSlot = false): a workgroup of P waves (4,
// or 8 on grids that leave CUs idle) per (kv-head, q-head chunk, request,
// split), the waves dealing the segment's tiles round-robin and merging
// through LDS. Slot-group (kSlot = true): one
// workgroup per (split, request) with one wave per kv-head (P = Hkv, groups of
// at most 16 q-heads), every wave walking every tile of the segment for its
// own head and writing its state directly. In the slot-group layout the waves
// of one CU read each cache slot (Hkv x 256 B) at about the same time; with
// the head-strided one the Hkv workgroups of a request run on different CUs,
// drift apart, and read a slot in 256-byte pieces at different times, which
// costs DRAM efficiency (measured on 64Q/8KV, S=32768, B=32: 637 vs 724 us).
template <int P, int T, bool kBlockUniform, bool kSlot = false>
__global__ __launch_bounds__(64 * P) void gqa_decode_mfma_kernel(const ScanArgs a) {
  const int lane = threadIdx.x & 63;
  const int ph = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15;   // MFMA column: q-head (QK), dim (PV)
  const int g = lane >> 4;   // MFMA row group
  const int hkv = kSlot ? ph : (int)blockIdx.x / a.nchunk;
  const int hc = kSlot ? 0 : (int)blockIdx.x - hkv * a.nchunk;
  const int b = blockIdx.y, split = kSlot ? blockIdx.x : blockIdx.z;
  const int h0 = hkv * a.G + hc * kMHeads;
  const int nh = min(kMHeads, a.G - hc * kMHeads);

  const int S = max(a.seq_lens[b], 0);
  const int ns = a.num_splits;
  const int chunk = ((S + ns - 1) / ns + 31) & ~31;
  const int seg_start = min(split * chunk, S);
  const int seg_end = min(S, seg_start + chunk);

  uint4 qf[4];
  mfma_load_q(a, b, h0, nh, j, g, qf);
  MfmaState st;
  mfma_init(st);
  __shared__ __attribute__((aligned(16))) uint8_t vlds_all[P][T * 256];
  mfma_scan_segment<T, kBlockUniform>(a, a.block_table + (size_t)b * a.max_blocks, hkv, qf,
                                      seg_start, seg_end, kSlot ? 0 : ph, kSlot ? 1 : P,
                                      vlds_all[ph], j, g, st);
  const f32x4_t(&o)[8] = st.o;
  // Lane (j, g) holds O rows of heads 4g + e; fetch their m and l.
  float Me[4], Le[4];
  mfma_finish(st, g, Me, Le);

  if constexpr (P == 1 || kSlot) {  // the wave holds its head's whole state
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int h = 4 * g + e;
      if (h >= nh) continue;
      const size_t bh = (size_t)b * a.Hq + h0 + h;
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) {
        if (a.out)
          a.out[bh * kHeadDim + 16 * nb + j] = (uint16_t)f32_to_bf16_bits(finalize(o[nb][e], Le[e]));
        if (a.ws_acc)
          put_state(a.ws_acc + (bh * ns + split) * kHeadDim + 16 * nb + j, o[nb][e], a.counters);
      }
      if (a.ws_acc && j == 0) {
        put_state(a.ws_m + bh * ns + split, Me[e] * kLn2, a.counters);
        put_state(a.ws_l + bh * ns + split, Le[e], a.counters);
      }
    }
  } else {
    // P waves share the kv-head: merge their states through LDS in wave order.
    __shared__ float lds_m[P][kMHeads];
    __shared__ float lds_l[P][kMHeads];
    __shared__ float lds_o[P][kMHeads][kHeadDim];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) lds_o[ph][4 * g + e][16 * nb + j] = o[nb][e];
      if (j == 0) {
        lds_m[ph][4 * g + e] = Me[e];
        lds_l[ph][4 * g + e] = Le[e];
      }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < nh * kHeadDim; idx += 64 * P) {
      const int h = idx / kHeadDim, d = idx % kHeadDim;
      float M = lds_m[0][h];
#pragma unroll
      for (int w = 1; w < P; ++w) M = fmaxf(M, lds_m[w][h]);
      const float Ms = M == kNegInf ? 0.f : M;
      float Lm = 0.f, A = 0.f;
#pragma unroll
      for (int w = 0; w < P; ++w) {
        const float mw = lds_m[w][h];
        const float f = mw == M ? 1.f : exp2_fast(mw - Ms);
        if (w == 0) {
          Lm = lds_l[0][h] * f;
          A = lds_o[0][h][d] * f;
        } else {
          Lm = fmaf(lds_l[w][h], f, Lm);
          A = fmaf(lds_o[w][h][d], f, A);
        }
      }
      const size_t bh = (size_t)b * a.Hq + h0 + h;
      if (a.out) a.out[bh * kHeadDim + d] = (uint16_t)f32_to_bf16_bits(finalize(A, Lm));
      if (a.ws_acc) {
        const size_t st = bh * ns + split;
        put_state(a.ws_acc + st * kHeadDim + d, A, a.counters);
        if (d == 0) {
          put_state(a.ws_m + st, M * kLn2, a.counters);
          put_state(a.ws_l + st, Lm, a.counters);
        }
      }
    }
  }
  // Single-launch split mode: the group's last workgroup merges its heads,
  // four per wave at a time. Slot-group layout: the group is the request and
  // each wave merges its own kv-head's q-heads; head-strided: the P waves
  // share the group's (at most 16) q-heads.
  if (a.counters != nullptr &&
      arrive_last(a.counters, kSlot ? (size_t)b : (size_t)b * gridDim.x + blockIdx.x, ns)) {
    const int first = kSlot ? 0 : 4 * ph, step = kSlot ? 4 : 4 * P;
    for (int h = first; h < nh; h += step)
      merge_heads4(a.ws_acc, a.ws_m, a.ws_l, a.merge_out, (size_t)b * a.Hq + h0 + h,
                   min(4, nh - h), ns, lane);
  }
}

template <int P, bool kSlot = false>
hipError_t launch_mfma_shape(const ScanArgs& a, dim3 grid, hipStream_t stream) {
  if (a.block_size % 16 == 0)
    hipLaunchKernelGGL((gqa_decode_mfma_kernel<P, kMTile, true, kSlot>), grid, dim3(64 * P), 0,
                       stream, a);
  else
    hipLaunchKernelGGL((gqa_decode_mfma_kernel<P, kMTile, false, kSlot>), grid, dim3(64 * P), 0,
                       stream, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_scan_mfma(const ScanArgs& args, int B, hipStream_t stream) {
  ScanArgs a = args;
  a.nchunk = (a.G + kMHeads - 1) / kMHeads;
  if (use_mfma_slot(B, a.Hkv, a.G, a.num_splits, device_cu_count())) {
    const dim3 grid(a.num_splits, B);
    if (a.Hkv == 4) return launch_mfma_shape<4, true>(a, grid, stream);
    return launch_mfma_shape<8, true>(a, grid, stream);
  }
  // Head-strided: 8 waves per split on grids that leave CUs idle (12 would
  // spill: the kernel needs ~180 VGPRs, and 3 waves per SIMD leave 168).
  const dim3 grid(a.Hkv * a.nchunk, B, a.num_splits);
  switch (waves_per_split((int64_t)B * a.Hkv * a.nchunk, a.num_splits,
                          (int64_t)a.max_blocks * a.block_size, kMWavesPerHead, 8,
                          device_cu_count())) {
    case 8: return launch_mfma_shape<8>(a, grid, stream);
    default: return launch_mfma_shape<kMWavesPerHead>(a, grid, stream);
  }
}

}  // namespace gqa
