// Issue-rate probes of one MI355X CU, behind the MLA decode's design choices
// (bench/issue_probe.py prints them; not on any decode path):
//   mfma    v_mfma_f32_16x16x32_bf16 throughput with 1..8 independent
//           accumulator chains per wave, one or two waves per SIMD;
//   overlap the same MFMA stream with NV independent v_fma_f32 per four
//           MFMAs, from one wave per SIMD (does a wave overlap its own VALU
//           work with its MFMAs?) and from two (does it overlap the other
//           wave's?);
//   lds     ds_read_b128 bandwidth per CU from 4 or 8 waves, conflict-free
//           addresses;
//   lanes   the lane semantics of gfx950's row-exchange instructions
//           (v_permlane16_swap_b32, v_permlane32_swap_b32), which the decode
//           kernels' cross-row reductions use (issue_probe_lane_swaps).
// Each probe is one launch of one workgroup per CU, timed with HIP events
// (median of 5); wave 0 of workgroup 0 also records the shader clock over its
// loop (s_memtime against the 100 MHz s_memrealtime). Every access stays
// inside its buffer: out holds one float per thread of the largest launch.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <vector>

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kMaxThreads = 512;
constexpr int kLdsBytes = 65536;

__device__ unsigned long long g_clock[2];  // wave 0's s_memtime and s_memrealtime deltas

// CH independent 16x16x32 chains (none if !MF) and NV independent FMAs per
// iteration.
template <int CH, int NV, bool MF>
__global__ __launch_bounds__(kMaxThreads) void mix_kernel(float* out, int iters, float s) {
  f32x4_t c[CH];
  for (int i = 0; i < CH; ++i) c[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float v[8];
  for (int i = 0; i < 8; ++i) v[i] = threadIdx.x * 0.001f + i;
  const u32x4_t ua = {threadIdx.x, 1u, 2u, 3u}, ub = {threadIdx.x ^ 5u, 7u, 9u, 11u};
  const bf16x8_t a = __builtin_bit_cast(bf16x8_t, ua), b = __builtin_bit_cast(bf16x8_t, ub);
  const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
    if constexpr (MF) {
#pragma unroll
      for (int i = 0; i < CH; ++i) c[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c[i], 0, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < NV; ++k) v[k & 7] = fmaf(v[k & 7], s, 1.0f);
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  float acc = 0.f;
  for (int i = 0; i < CH; ++i) acc += c[i][0] + c[i][1] + c[i][2] + c[i][3];
  for (int i = 0; i < 8; ++i) acc += v[i];
  out[blockIdx.x * blockDim.x + threadIdx.x] = acc;
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    g_clock[0] = t1 - t0;
    g_clock[1] = r1 - r0;
  }
}

// NR ds_read_b128 in flight per wave, linear addresses (conflict-free).
template <int NR>
__global__ __launch_bounds__(kMaxThreads) void lds_kernel(float* out, int iters) {
  __shared__ __attribute__((aligned(16))) uint8_t sm[kLdsBytes];
  for (int i = threadIdx.x; i < kLdsBytes / 4; i += blockDim.x) reinterpret_cast<uint32_t*>(sm)[i] = i;
  __syncthreads();
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  uint32_t base = (uint32_t)((w * 4096 + lane * 16) & (kLdsBytes - 1));
  u32x4_t acc = {0u, 0u, 0u, 0u};
  for (int it = 0; it < iters; ++it) {
    u32x4_t r[NR];
#pragma unroll
    for (int k = 0; k < NR; ++k)
      r[k] = *reinterpret_cast<const u32x4_t*>(sm + ((base + 1024 * k) & (kLdsBytes - 1)));
#pragma unroll
    for (int k = 0; k < NR; ++k) acc ^= r[k];
    base = (base + 1024 * NR) & (kLdsBytes - 1);
  }
  out[blockIdx.x * blockDim.x + threadIdx.x] = (float)(acc[0] ^ acc[1] ^ acc[2] ^ acc[3]);
}

// The first HIP error of a probe run (checked by issue_probe_run at its end).
hipError_t g_error = hipSuccess;
void note(hipError_t e) {
  if (e != hipSuccess && g_error == hipSuccess) g_error = e;
}

template <typename F>
float median_ms(F launch) {
  hipEvent_t e0, e1;
  note(hipEventCreate(&e0));
  note(hipEventCreate(&e1));
  launch();
  note(hipDeviceSynchronize());
  std::vector<float> ts;
  for (int r = 0; r < 5; ++r) {
    note(hipEventRecord(e0));
    launch();
    note(hipEventRecord(e1));
    note(hipEventSynchronize(e1));
    float ms = 0.f;
    note(hipEventElapsedTime(&ms, e0, e1));
    ts.push_back(ms);
  }
  note(hipEventDestroy(e0));
  note(hipEventDestroy(e1));
  std::sort(ts.begin(), ts.end());
  return ts[2];
}

double clock_mhz() {
  unsigned long long c[2] = {0, 0};
  note(hipMemcpyFromSymbol(c, HIP_SYMBOL(g_clock), sizeof(c)));
  return c[1] ? 100.0 * (double)c[0] / (double)c[1] : 0.0;
}

// One wave, x = lane id: out[0..63] and out[64..127] are the two results of
// v_permlane16_swap_b32 with x as both operands, out[128..191] and
// out[192..255] those of v_permlane32_swap_b32.
__global__ __launch_bounds__(64) void lane_swap_kernel(uint32_t* out) {
  const uint32_t x = threadIdx.x;
  const auto a = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  out[x] = a[0];
  out[64 + x] = a[1];
  out[128 + x] = b[0];
  out[192 + x] = b[1];
}

}  // namespace

// Runs lane_swap_kernel once and copies its 256 results to host_out. Returns 0,
// or -1 on a HIP error.
extern "C" __attribute__((visibility("default"))) int issue_probe_lane_swaps(uint32_t* host_out) {
  uint32_t* out = nullptr;
  if (hipMalloc(&out, 256 * sizeof(uint32_t)) != hipSuccess) return -1;
  lane_swap_kernel<<<1, 64>>>(out);
  hipError_t err = hipGetLastError();
  if (err == hipSuccess) err = hipMemcpy(host_out, out, 256 * sizeof(uint32_t), hipMemcpyDeviceToHost);
  const hipError_t free_err = hipFree(out);
  return err == hipSuccess && free_err == hipSuccess ? 0 : -1;
}

// Runs every probe on `cus` workgroups (one per CU) and writes, per probe,
// {kind, chains or reads in flight, FMAs per iteration, threads, ms, clock MHz}
// as 6 doubles to rows (at most max_rows). Returns the number of rows, or -1 on
// a HIP error. kind: 0 mfma/overlap, 1 lds.
extern "C" __attribute__((visibility("default"))) int issue_probe_run(double* rows, int max_rows,
                                                                     int cus, int iters) {
  float* out = nullptr;
  if (hipMalloc(&out, sizeof(float) * (size_t)cus * kMaxThreads) != hipSuccess) return -1;
  g_error = hipSuccess;
  int n = 0;
  auto put = [&](double kind, double p1, double p2, double thr, double ms, double mhz) {
    if (n >= max_rows) return;
    double* r = rows + 6 * n++;
    r[0] = kind; r[1] = p1; r[2] = p2; r[3] = thr; r[4] = ms; r[5] = mhz;
  };
#define MIX(CH, NV, MF, THR)                                                                      \
  {                                                                                               \
    const float ms = median_ms([&] { mix_kernel<CH, NV, MF><<<cus, THR>>>(out, iters, 0.999f); }); \
    put(0, MF ? CH : 0, NV, THR, ms, clock_mhz());                                                \
  }
  MIX(1, 0, true, 256) MIX(2, 0, true, 256) MIX(4, 0, true, 256) MIX(8, 0, true, 256)
  MIX(4, 0, true, 512)
  MIX(4, 8, false, 256) MIX(4, 16, false, 256)
  MIX(4, 4, true, 256) MIX(4, 8, true, 256) MIX(4, 16, true, 256)
  MIX(4, 8, false, 512) MIX(4, 4, true, 512) MIX(4, 8, true, 512)
#undef MIX
  for (int thr : {256, 512}) {
    const float ms4 = median_ms([&] { lds_kernel<4><<<cus, thr>>>(out, iters); });
    put(1, 4, 0, thr, ms4, 0.0);
    const float ms8 = median_ms([&] { lds_kernel<8><<<cus, thr>>>(out, iters); });
    put(1, 8, 0, thr, ms8, 0.0);
  }
  note(hipGetLastError());
  note(hipFree(out));
  return g_error == hipSuccess ? n : -1;
}
