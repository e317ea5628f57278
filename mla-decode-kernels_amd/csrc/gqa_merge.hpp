// Log-sum-exp merge of split states (v2_splitkv.cu:92-108) for the merge
// kernel (merge_head) and for the single-launch split kernels, whose last
// workgroup of each group folds the group's states itself (merge_heads4).
// Both apply the same operations to every output element in the same order,
// so a fused launch and a partial + merge pair give the same bits.
#pragma once

#include "gqa_device.hpp"

namespace gqa {

// Split states that another workgroup of the same launch reads (single-launch
// split mode) are stored and loaded at device scope: the stores write through
// to the level every XCD reads from, the loads skip cached copies. Their
// ordering against the arrival count is arrive_last's release/acquire pair.
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Two consecutive floats (8-byte aligned) in one device-scope access.
__device__ __forceinline__ void store_coherent2(float* p, float a, float b) {
  const uint64_t v = (uint64_t)__float_as_uint(a) | ((uint64_t)__float_as_uint(b) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 load_coherent2(const float* p) {
  const uint64_t v = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__uint_as_float((uint32_t)v), __uint_as_float((uint32_t)(v >> 32)));
}

// One split's term in the log-sum-exp fold of an output element (the
// reference's merge, v2_splitkv.cu:92-108): with M the max of the element's
// split maxima (natural-log units), split i's factor is f = e^(m_i - M),
// exactly 1 for a split holding the max and 0 for an empty split
// (m_i = -inf); the first split sets L = l_i f and A = acc_i f, every later one
// adds l_i f and acc_i f with a fused multiply-add. Every merge in this library
// (the merge kernel, the single-launch merges, the in-workgroup merge) folds
// each element with these two steps, in split order, so all give the same
// bits.
__device__ __forceinline__ float fold_factor(float mi, float M) {
  return mi == M ? 1.f : exp2_fast((mi - M) * kLog2e);
}
__device__ __forceinline__ void fold_term(bool first, float x, float f, float& acc) {
  acc = first ? x * f : fmaf(x, f, acc);
}

// One wave folds the ns states of (b, q-head) bh, stored at state index
// bh * ns + i (the reference's [B, Hq, ns] layout), and writes out's row bh:
// lane i owns dims {2i, 2i + 1}. The splits are folded in index order,
// kBatch at a time: a batch's acc rows are loaded together, and its m and l
// with one load each (lane k holds split i0 + k's, broadcast with
// v_readlane). The first batch's loads are issued together with the loads of
// the maxima (one split per lane), so at most kBatch splits take one memory
// round trip. The factor of the split holding the max is exactly 1, so one
// split merges to itself bit for bit.
template <int kBatch>
__device__ __forceinline__ void merge_head(const float* __restrict__ ws_acc,
                                           const float* __restrict__ ws_m,
                                           const float* __restrict__ ws_l,
                                           uint16_t* __restrict__ out, size_t bh, int ns,
                                           int lane) {
  static_assert(kBatch <= 64, "a batch's m and l are held one per lane");
  const size_t st0 = bh * ns;
  float mb, lb;  // lane k < kBatch: m and l of split i0 + k
  float2 av[kBatch];
  auto load_batch = [&](int i0) {
    // Past the end: a valid split, not folded.
    const size_t sl = st0 + min(i0 + (lane & (kBatch - 1)), ns - 1);
    mb = ws_m[sl];
    lb = ws_l[sl];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const size_t st = st0 + min(i0 + k, ns - 1);
      av[k] = reinterpret_cast<const float2*>(ws_acc + st * kHeadDim)[lane];
    }
  };
  load_batch(0);
  float mloc = kNegInf;
  for (int i = lane; i < ns; i += 64) mloc = fmaxf(mloc, ws_m[st0 + i]);
  const float M = wave_max(mloc);
  float L = 0.f, A0 = 0.f, A1 = 0.f;
  for (int i0 = 0; i0 < ns; i0 += kBatch) {
    if (i0 > 0) load_batch(i0);
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      if (i0 + k >= ns) break;
      const float mi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mb), k));
      const float li = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lb), k));
      const float f = fold_factor(mi, M);
      const bool first = i0 + k == 0;
      fold_term(first, li, f, L);
      fold_term(first, av[k].x, f, A0);
      fold_term(first, av[k].y, f, A1);
    }
  }
  const uint32_t lo = f32_to_bf16_bits(finalize(A0, L));
  const uint32_t hi = f32_to_bf16_bits(finalize(A1, L));
  reinterpret_cast<uint32_t*>(out + bh * kHeadDim)[lane] = lo | (hi << 16);
}

// A split state element: plain store, or device-scope when the launch merges
// in-kernel (coherent = the launch's counters, non-null).
__device__ __forceinline__ void put_state(float* p, float v, const void* coherent) {
  if (coherent)
    store_coherent(p, v);
  else
    *p = v;
}

// merge_head for up to four heads at once, bh0 .. bh0 + nheads - 1, reading
// the states at device scope: lane l serves head bh0 + l/16, dims
// 32j + 2(l%16) + {0, 1} for j < 4, so each 8-byte load of 16 lanes covers
// 128 contiguous bytes. Each output element sees the same operations in the
// same order as in merge_head (the max is exact in any order), so the two
// give the same bits.
__device__ __forceinline__ void merge_heads4(const float* __restrict__ ws_acc,
                                             const float* __restrict__ ws_m,
                                             const float* __restrict__ ws_l,
                                             uint16_t* __restrict__ out, size_t bh0, int nheads,
                                             int ns, int lane) {
  constexpr int kBatch = 8;
  const int hi = lane >> 4, c = lane & 15;
  const bool live = hi < nheads;
  const size_t st0 = (bh0 + (live ? hi : 0)) * ns;
  float mi[kBatch], li[kBatch], av[kBatch][8];
  auto load_batch = [&](int i0) {
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const size_t st = st0 + min(i0 + k, ns - 1);  // past the end: a valid split, not folded
      mi[k] = load_coherent(ws_m + st);
      li[k] = load_coherent(ws_l + st);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float2 x = load_coherent2(ws_acc + st * kHeadDim + 32 * j + 2 * c);
        av[k][2 * j] = x.x;
        av[k][2 * j + 1] = x.y;
      }
    }
  };
  load_batch(0);  // issued with the maxima's loads: one round trip for <= kBatch splits
  float mloc = kNegInf;
  for (int i = c; i < ns; i += 16) mloc = fmaxf(mloc, load_coherent(ws_m + st0 + i));
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) mloc = fmaxf(mloc, __shfl_xor(mloc, o, 64));
  const float M = mloc;
  float L = 0.f;
  float A[8];
#pragma unroll
  for (int d = 0; d < 8; ++d) A[d] = 0.f;
  for (int i0 = 0; i0 < ns; i0 += kBatch) {
    if (i0 > 0) load_batch(i0);
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      if (i0 + k >= ns) break;
      const float f = fold_factor(mi[k], M);
      const bool first = i0 + k == 0;
      fold_term(first, li[k], f, L);
#pragma unroll
      for (int d = 0; d < 8; ++d) fold_term(first, av[k][d], f, A[d]);
    }
  }
  if (live) {
    uint32_t* dst = reinterpret_cast<uint32_t*>(out + (bh0 + hi) * kHeadDim);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      dst[16 * j + c] = f32_to_bf16_bits(finalize(A[2 * j], L)) |
                        (f32_to_bf16_bits(finalize(A[2 * j + 1], L)) << 16);
  }
}

// Arrival of a workgroup at the end of its split for merge group `group`, with
// ns workgroups per group: the "last workgroup merges" protocol in its
// textbook form under the HIP (scoped C++) memory model, with each fence
// placed once.
//  - Every thread's state stores happen before thread 0's count: each thread
//    waits for its stores to complete (s_waitcnt vmcnt(0), gfx9 encoding) and
//    the workgroup meets at a barrier behind a workgroup-scope release fence.
//  - Thread 0 counts with a release read-modify-write at device (agent)
//    scope: on gfx950 the compiler emits an L2 writeback (buffer_wbl2 sc1)
//    and a store wait before the atomic, so the workgroup's states reach the
//    level every XCD reads before the count can be seen.
//  - The workgroup that sees ns - 1 arrivals takes an acquire fence at device
//    scope (buffer_inv sc1: this XCD's L2 drops non-local copies), which
//    synchronises with every earlier arrival's release; the barrier after it
//    passes that on to the workgroup's other threads. It sets the counter back
//    to zero: all ns arrivals of this launch are counted.
// The states themselves are also stored and loaded at device scope
// (write-through stores, loads that skip cached copies), so they leave no
// dirty lines for the writeback. Only one thread per workgroup pays for the
// writeback and only the last workgroup of a group for the invalidate; a
// device-scope fence in every wave instead (each would do both) made config 2
// at 8 splits 3.3x slower. Returns, in every thread, whether this workgroup
// arrived last. Nothing waits on another workgroup. Call from every thread of
// the workgroup, after its state stores.
__device__ __forceinline__ bool arrive_last(uint32_t* counters, size_t group, int ns) {
  __shared__ uint32_t last_flag;
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(counters + group, 1u, __ATOMIC_RELEASE,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    const bool last = prev == (uint32_t)(ns - 1);
    if (last) {
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      __hip_atomic_store(counters + group, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    last_flag = last ? 1u : 0u;
  }
  __syncthreads();
  const bool last = last_flag != 0;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  return last;
}

}  // namespace gqa
