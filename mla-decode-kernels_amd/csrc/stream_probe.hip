// Streaming-read probe: the HBM read rate of the decode scans' access pattern
// with no arithmetic, the measured ceiling the scans are compared against.
// Measurement code (bench.py --stream-probe), built into its own library; the
// decode kernels do not use it.
//
// The cache is modelled as config 2 lays it out: K and V buffers of `requests`
// x `slots` token slots of 8 kv-heads x 256 bytes (a 2 KiB slot), each
// request's slots contiguous (an identity block table). Every byte of both
// buffers is read exactly once, with 16-byte buffer loads (non-temporal or
// plain), one tile of loads in flight per wave ahead of the one being folded,
// as the scans do. Three patterns:
//   head-strided  grid (8 kv-heads, requests) x 4 waves, the VALU scan's
//                 layout: the workgroup of kv-head h reads 256-byte head rows
//                 at the 2 KiB slot stride; a load instruction covers 4 slots
//                 (1 KiB), a tile is 16 slots (4 K + 4 V loads), the waves take
//                 tiles round-robin. Workgroups are mapped to kv-heads with
//                 adjacent heads swapped (h ^ 1), as the scan maps them.
//   whole-slot    grid (splits, requests) x 4 waves: each load instruction
//                 covers half a slot (1 KiB, 4 heads), a tile is 2 whole slots
//                 (4 K + 4 V loads), so a CU reads every slot it touches whole.
//   linear        256 workgroups x 4 waves (one wave per SIMD) stream both
//                 buffers front to back: wave g of W takes 4 KiB chunks g,
//                 g + W, ... (4 K + 4 V loads of 1 KiB per chunk); the plain
//                 sequential read, with no gather at all. With fewer
//                 workgroups (4 or 16 waves each) than CUs it measures what
//                 the occupied CUs alone can stream.
//   paged         the head-strided pattern through a block table: 16-slot
//                 blocks (32 KiB) at the ids the table gives, as config 2's
//                 cache is read (gqa_stream_probe_paged_launch).
// Each lane folds what it loaded into one word written to `sink`, so no load
// is dead. Every pattern takes its wave index through readfirstlane, as the
// decode kernels do: derived from threadIdx alone, the index is not known to
// be wave-uniform, the tile loop's branches then run under exec masks, and
// their conservative load waits slowed the paged read from 157 to 181 us
// (identity table).
//
// The timed entry point (gqa_stream_probe_timed_launch) also records, per
// workgroup, the 100 MHz real-time counter at its start and end, which shows
// how much of a launch is its tail; it runs the head-strided pattern or a
// dynamic one:
//   dynamic       256 persistent workgroups x 4 waves; the items are
//                 (chunk, request, kv-head) triples of `chunk` slots, in
//                 chunk-major order (the first 256 are the head-strided
//                 pattern's workgroups' first chunks); workgroup g reads item g
//                 and then claims further items from a counter (a vector
//                 atomic by thread 0, one item ahead) until none are left.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kHeads = 8;
constexpr int kRowBytes = 256;
constexpr uint32_t kSlotBytes = kHeads * kRowBytes;  // 2 KiB

template <bool kNT>
__device__ __forceinline__ uint4 load16(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kNT ? 2 : 0));
}

__device__ __forceinline__ uint32_t fold(const uint4& a) { return a.x ^ a.y ^ a.z ^ a.w; }

// Reads the wave's tiles k = 0 .. my - 1 (tile k: loads off(k, i) of K and V
// for i < 4), one tile ahead; returns the lane's fold.
template <bool kNT, typename Off>
__device__ __forceinline__ uint32_t stream_tiles(__amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv,
                                                 int my, Off off) {
  uint32_t acc = 0;
  uint4 t[2][8];
  auto issue = [&](int k, uint4 (&d)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      d[i] = load16<kNT>(rk, off(k, i));
      d[4 + i] = load16<kNT>(rv, off(k, i));
    }
  };
  if (my > 0) issue(0, t[0]);
  for (int k = 0; k < my; k += 2) {
    if (k + 1 < my) issue(k + 1, t[1]);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc += fold(t[0][i]);
    if (k + 1 >= my) break;
    if (k + 2 < my) issue(k + 2, t[0]);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc += fold(t[1][i]);
  }
  return acc;
}

// The wave's share of ntiles tiles dealt round-robin over 4 waves: tiles ph,
// ph + 4, ...
__device__ __forceinline__ int round_robin_count(int ntiles, int ph) {
  return ntiles > ph ? (ntiles - ph + 3) / 4 : 0;
}

// The workgroup's start and end on the 100 MHz real-time counter, by thread 0
// after a barrier (every wave's loads have been folded by then).
__device__ __forceinline__ void record_times(unsigned long long* times, int wg,
                                             unsigned long long t0) {
  if (times == nullptr) return;
  __syncthreads();
  if (threadIdx.x == 0) {
    times[2 * wg] = t0;
    times[2 * wg + 1] = __builtin_amdgcn_s_memrealtime();
  }
}

template <bool kNT>
__global__ __launch_bounds__(256) void probe_head_strided(const uint8_t* K, const uint8_t* V,
                                                          uint32_t* sink, int slots,
                                                          unsigned long long* times) {
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  const int h = blockIdx.x ^ 1, b = blockIdx.y;
  const int lane = threadIdx.x & 63, ph = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane >> 4, c = lane & 15;
  const size_t base = (size_t)b * slots * kSlotBytes;
  const uint32_t bytes = (uint32_t)slots * kSlotBytes;
  const auto rk = __builtin_amdgcn_make_buffer_rsrc((void*)(K + base), 0, bytes, 0x00020000);
  const auto rv = __builtin_amdgcn_make_buffer_rsrc((void*)(V + base), 0, bytes, 0x00020000);
  const uint32_t acc = stream_tiles<kNT>(rk, rv, round_robin_count(slots / 16, ph), [&](int k, int i) {
    return (uint32_t)(16 * (ph + 4 * k) + 4 * i + r) * kSlotBytes + h * kRowBytes + 16 * c;
  });
  sink[((size_t)b * gridDim.x + blockIdx.x) * 256 + threadIdx.x] = acc;
  record_times(times, b * gridDim.x + blockIdx.x, t0);
}

// Dynamic: `requests` x 8 x (slots / chunk) items of `chunk` slots (see the
// file comment); ctr[0] counts claims and ctr[1] departures, both zero on
// entry; the last workgroup to leave sets them back to zero.
__global__ __launch_bounds__(256) void probe_dynamic(const uint8_t* K, const uint8_t* V,
                                                     uint32_t* sink, int requests, int slots,
                                                     int chunk, unsigned int* ctr,
                                                     unsigned long long* times) {
  __shared__ int next_item[2];
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  const int lane = threadIdx.x & 63, ph = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane >> 4, c = lane & 15;
  const int per_chunk = requests * kHeads, nitems = per_chunk * (slots / chunk);
  uint32_t acc = 0;
  int item = blockIdx.x, par = 0;
  while (item < nitems) {
    int claimed = 0;
    if (threadIdx.x == 0)
      claimed = (int)__hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) +
                (int)gridDim.x;
    const int ck = item / per_chunk, bh = item - ck * per_chunk;
    const int b = bh / kHeads, h = (bh % kHeads) ^ 1;
    const size_t base = ((size_t)b * slots + (size_t)ck * chunk) * kSlotBytes;
    const uint32_t bytes = (uint32_t)chunk * kSlotBytes;
    const auto rk = __builtin_amdgcn_make_buffer_rsrc((void*)(K + base), 0, bytes, 0x00020000);
    const auto rv = __builtin_amdgcn_make_buffer_rsrc((void*)(V + base), 0, bytes, 0x00020000);
    acc += stream_tiles<true>(rk, rv, round_robin_count(chunk / 16, ph), [&](int k, int i) {
      return (uint32_t)(16 * (ph + 4 * k) + 4 * i + r) * kSlotBytes + h * kRowBytes + 16 * c;
    });
    if (threadIdx.x == 0) next_item[par] = claimed;
    __syncthreads();
    item = next_item[par];
    par ^= 1;
  }
  sink[(size_t)blockIdx.x * 256 + threadIdx.x] = acc;
  record_times(times, blockIdx.x, t0);
  if (threadIdx.x == 0) {
    const uint32_t left = __hip_atomic_fetch_add(ctr + 1, 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    if (left == gridDim.x - 1) {
      __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(ctr + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

template <bool kNT>
__global__ __launch_bounds__(256) void probe_whole_slot(const uint8_t* K, const uint8_t* V,
                                                        uint32_t* sink, int slots) {
  const int sp = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x & 63, ph = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int per = slots / gridDim.x;
  const size_t base = ((size_t)b * slots + (size_t)sp * per) * kSlotBytes;
  const uint32_t bytes = (uint32_t)per * kSlotBytes;
  const auto rk = __builtin_amdgcn_make_buffer_rsrc((void*)(K + base), 0, bytes, 0x00020000);
  const auto rv = __builtin_amdgcn_make_buffer_rsrc((void*)(V + base), 0, bytes, 0x00020000);
  const uint32_t acc = stream_tiles<kNT>(rk, rv, round_robin_count(per / 2, ph), [&](int k, int i) {
    return (uint32_t)(2 * (ph + 4 * k) + (i >> 1)) * kSlotBytes + (i & 1) * 1024u + 16 * lane;
  });
  sink[((size_t)b * gridDim.x + blockIdx.x) * 256 + threadIdx.x] = acc;
}

template <bool kNT, int W = 4>
__global__ __launch_bounds__(64 * W) void probe_linear(const uint8_t* K, const uint8_t* V,
                                                       uint32_t* sink, uint32_t bytes) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * W + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int waves = gridDim.x * W;
  const auto rk = __builtin_amdgcn_make_buffer_rsrc((void*)K, 0, bytes, 0x00020000);
  const auto rv = __builtin_amdgcn_make_buffer_rsrc((void*)V, 0, bytes, 0x00020000);
  const int chunks = (int)(bytes / 4096u);
  const int mine = chunks > wave ? (chunks - wave + waves - 1) / waves : 0;
  const uint32_t acc = stream_tiles<kNT>(rk, rv, mine, [&](int k, int i) {
    return (uint32_t)(wave + waves * k) * 4096u + (uint32_t)i * 1024u + 16u * lane;
  });
  sink[(size_t)blockIdx.x * 64 * W + threadIdx.x] = acc;
}

// Paged head-strided: the head-strided pattern over a paged cache. K and V
// are pools of 16-slot blocks (32 KiB each, slots of 8 kv-heads x 256 B);
// request b's tile k (16 tokens) is block bt[b * nblk + k], its id read as a
// scalar through the constant address space, as the VALU scan reads it from
// its block table. With a shuffled table this is config 2's access pattern
// (block size 16) without the scan's arithmetic.
__global__ __launch_bounds__(256) void probe_paged(const uint8_t* K, const uint8_t* V,
                                                   const int* bt, uint32_t* sink, int nblk) {
  const int h = blockIdx.x ^ 1, b = blockIdx.y;
  const int lane = threadIdx.x & 63, ph = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane >> 4, c = lane & 15;
  const auto* btc = (const __attribute__((address_space(4))) int*)(bt + (size_t)b * nblk);
  const int my = round_robin_count(nblk, ph);
  const uint32_t bytes = 16 * kSlotBytes - (uint32_t)h * kRowBytes;
  uint32_t acc = 0;
  uint4 t[2][8];
  auto issue = [&](int k, uint4 (&d)[8]) {
    const size_t base = (size_t)btc[ph + 4 * k] * (16 * kSlotBytes) + (size_t)h * kRowBytes;
    const auto rk = __builtin_amdgcn_make_buffer_rsrc((void*)(K + base), 0, bytes, 0x00020000);
    const auto rv = __builtin_amdgcn_make_buffer_rsrc((void*)(V + base), 0, bytes, 0x00020000);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t off = (uint32_t)(4 * i + r) * kSlotBytes + 16 * c;
      d[i] = load16<true>(rk, off);
      d[4 + i] = load16<true>(rv, off);
    }
  };
  if (my > 0) issue(0, t[0]);
  for (int k = 0; k < my; k += 2) {
    if (k + 1 < my) issue(k + 1, t[1]);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc += fold(t[0][i]);
    if (k + 1 >= my) break;
    if (k + 2 < my) issue(k + 2, t[0]);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc += fold(t[1][i]);
  }
  sink[((size_t)b * gridDim.x + blockIdx.x) * 256 + threadIdx.x] = acc;
}

}  // namespace

// Paged head-strided read (non-temporal loads): K and V are pools of
// requests * nblk blocks of 16 slots (32 KiB each), bt an int32 table
// [requests, nblk] of block ids in [0, requests * nblk); grid (8 kv-heads,
// requests) x 4 waves. sink holds requests * 8 * 256 words. Returns
// hipErrorInvalidValue for a null pointer, requests outside [1, 65535] or
// nblk < 1, else the launch status. The ids are not checked: every one must
// lie in the pool.
extern "C" __attribute__((visibility("default"))) int gqa_stream_probe_paged_launch(
    const void* k, const void* v, const int* bt, uint32_t* sink, int requests, int nblk,
    hipStream_t stream) {
  if (!k || !v || !bt || !sink || requests < 1 || requests > 65535 || nblk < 1)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(probe_paged, dim3(kHeads, requests), dim3(256), 0, stream,
                     static_cast<const uint8_t*>(k), static_cast<const uint8_t*>(v), bt, sink,
                     nblk);
  return hipGetLastError();
}

// Reads K and V ([requests, slots, 8 heads, 256 B] each) once in `pattern`
// (0 head-strided, 1 whole-slot with `splits` workgroups per request, 2 linear
// with `splits` workgroups in all, 4 linear with `splits` workgroups of 16
// waves: with fewer workgroups than CUs, the most one CU streams) with
// non-temporal (nontemporal != 0) or plain loads. sink holds one word per
// thread: requests * 8 * 256 words for pattern 0, requests * splits * 256 for
// pattern 1, splits * 256 for pattern 2, splits * 1024 for pattern 4. Requires slots % 64 == 0 (pattern 1: slots % (2 * splits) == 0), slots *
// 2 KiB < 4 GiB (pattern 2: the whole buffer). Returns hipErrorInvalidValue for
// other arguments, else the launch status.
extern "C" __attribute__((visibility("default"))) int gqa_stream_probe_launch(
    const void* k, const void* v, uint32_t* sink, int pattern, int requests, int slots, int splits,
    int nontemporal, hipStream_t stream) {
  if (!k || !v || !sink || requests < 1 || requests > 65535 || slots < 64 || slots % 64 != 0 ||
      (uint64_t)slots * kSlotBytes >= (uint64_t(1) << 32))
    return hipErrorInvalidValue;
  const auto* K = static_cast<const uint8_t*>(k);
  const auto* V = static_cast<const uint8_t*>(v);
  if (pattern == 0) {
    const dim3 grid(kHeads, requests);
    if (nontemporal)
      hipLaunchKernelGGL(probe_head_strided<true>, grid, dim3(256), 0, stream, K, V, sink, slots,
                         nullptr);
    else
      hipLaunchKernelGGL(probe_head_strided<false>, grid, dim3(256), 0, stream, K, V, sink, slots,
                         nullptr);
  } else if (pattern == 1) {
    if (splits < 1 || splits > 65535 || slots % (2 * splits) != 0) return hipErrorInvalidValue;
    const dim3 grid(splits, requests);
    if (nontemporal)
      hipLaunchKernelGGL(probe_whole_slot<true>, grid, dim3(256), 0, stream, K, V, sink, slots);
    else
      hipLaunchKernelGGL(probe_whole_slot<false>, grid, dim3(256), 0, stream, K, V, sink, slots);
  } else if (pattern == 2 || pattern == 4) {
    const uint64_t bytes = (uint64_t)requests * slots * kSlotBytes;
    if (splits < 1 || splits > 65535 || bytes >= (uint64_t(1) << 32)) return hipErrorInvalidValue;
    if (pattern == 4 && nontemporal)
      hipLaunchKernelGGL((probe_linear<true, 16>), dim3(splits), dim3(1024), 0, stream, K, V, sink,
                         (uint32_t)bytes);
    else if (pattern == 4)
      hipLaunchKernelGGL((probe_linear<false, 16>), dim3(splits), dim3(1024), 0, stream, K, V,
                         sink, (uint32_t)bytes);
    else if (nontemporal)
      hipLaunchKernelGGL(probe_linear<true>, dim3(splits), dim3(256), 0, stream, K, V, sink,
                         (uint32_t)bytes);
    else
      hipLaunchKernelGGL(probe_linear<false>, dim3(splits), dim3(256), 0, stream, K, V, sink,
                         (uint32_t)bytes);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Timed runs (non-temporal loads): pattern 0 head-strided (grid 8 x requests),
// pattern 3 dynamic (256 workgroups, items of `chunk` slots). times receives
// (start, end) per workgroup on the 100 MHz real-time counter: 8 * requests
// pairs for pattern 0, 256 for pattern 3. ctr (pattern 3): two 32-bit
// counters, zero before the first launch and left zero by each. sink: one word
// per thread (8 * requests * 256 words suffice for both). Same size rules as
// above; pattern 3 also needs 16 <= chunk, slots % chunk == 0 and chunk % 16 == 0.
extern "C" __attribute__((visibility("default"))) int gqa_stream_probe_timed_launch(
    const void* k, const void* v, uint32_t* sink, unsigned long long* times, unsigned int* ctr,
    int pattern, int requests, int slots, int chunk, hipStream_t stream) {
  if (!k || !v || !sink || !times || requests < 1 || requests > 65535 || slots < 64 ||
      slots % 64 != 0 || (uint64_t)slots * kSlotBytes >= (uint64_t(1) << 32))
    return hipErrorInvalidValue;
  const auto* K = static_cast<const uint8_t*>(k);
  const auto* V = static_cast<const uint8_t*>(v);
  if (pattern == 0) {
    hipLaunchKernelGGL(probe_head_strided<true>, dim3(kHeads, requests), dim3(256), 0, stream, K,
                       V, sink, slots, times);
  } else if (pattern == 3) {
    if (!ctr || chunk < 16 || chunk % 16 != 0 || slots % chunk != 0 || requests * kHeads < 256)
      return hipErrorInvalidValue;
    hipLaunchKernelGGL(probe_dynamic, dim3(256), dim3(256), 0, stream, K, V, sink, requests, slots,
                       chunk, ctr, times);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
