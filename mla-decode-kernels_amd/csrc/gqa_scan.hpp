// Arguments and launch entry points shared by the two scan kernels (VALU
// single-pass/partial kernel and the MFMA one).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gqa_device.hpp"

namespace gqa {

struct ScanArgs {
  const uint16_t* q;
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  const int* block_table;
  const int* seq_lens;
  uint16_t* out;  // single-pass mode: normalised bf16 output (num_splits == 1)
  float* ws_acc;  // split mode: unnormalised per-split state
  float* ws_m;
  float* ws_l;
  int Hq, Hkv, G, nchunk, block_size, max_blocks, num_splits;
  FastDiv bs_div;
  float scale_log2e;  // scale * log2(e): scores are kept in base-2 units
  // Single-launch split mode: one arrival counter per merge group (zero on
  // entry, left zero), and the output the group's last workgroup writes.
  uint32_t* counters = nullptr;
  uint16_t* merge_out = nullptr;
};

// The kv-head a head-strided VALU-scan workgroup (or a token-balanced VALU
// segment) serves, from its grid position (segment ordinal) x: adjacent
// heads swapped when Hkv is even. Workgroups are dealt
// round-robin to the 8 XCDs by linear id, and with an even grid x extent the
// XCD number has the parity of x; a head's 256-byte rows have address bit 8
// equal to the head's parity. On MI355X the VALU scan's gather streams faster
// when each XCD reads heads of the other parity (probe, 1 GiB: 154.5 us
// against 161 us; config 2: 164.3 vs 166.2 us, config 3: 165.6 vs 169.2). The
// matrix-core scan's head-strided launch, which loads K in 64-byte row
// pieces, was 1-2 % slower with the swap and keeps the plain order. The swap
// only changes which workgroup computes a (request, kv-head) pair, not how, so
// results are unchanged bit for bit.
__device__ __forceinline__ int strided_kv_head(int x, int Hkv) {
  return (Hkv & 1) ? x : (x ^ 1);
}

// GQA groups of at least this many q-heads run the matrix-core scan
// (gqa_scan_mfma.hpp): its VALU work per tile does not grow with the group,
// while the VALU scan's does (measured: 8-head groups are VALU-bound on the
// VALU scan at ~60% of HBM peak; 4-head groups stream ~5% faster there).
#ifndef GQA_MFMA_MIN_GROUP
#define GQA_MFMA_MIN_GROUP 5
#endif
inline bool use_mfma(int G) { return G >= GQA_MFMA_MIN_GROUP; }

// The matrix-core scan's slot-group layout (one workgroup of Hkv waves per
// (split, request), one wave per kv-head) serves groups of at most 16 q-heads
// with 4 or 8 kv-heads (16 would make 16-wave workgroups, whose register
// budget spills) when the grid gives at least 3/4 of the CUs their full
// residency of 8 waves (two per SIMD, which hides the scan's per-tile
// dependency chain).
inline bool mfma_slot_shape(int Hkv, int G) { return G <= 16 && (Hkv == 4 || Hkv == 8); }
inline bool use_mfma_slot(int B, int Hkv, int G, int num_splits, int num_cus) {
  return mfma_slot_shape(Hkv, G) && num_cus > 0 &&
         (int64_t)B * num_splits * Hkv * 4 >= (int64_t)24 * num_cus;
}

// Waves per split of a head-strided launch of `wgs` workgroups per split
// index (requests x kv-heads x head chunks) over splits of a sequence of up
// to s_max tokens: `base`, or the largest of 8, 12 and 16 (at most max_p)
// that keeps the whole grid within one wave per SIMD of the device and gives
// every wave at least two 16-token tiles of the longest split. Only a grid
// that leaves CUs idle takes more than `base`: a workgroup streams through
// its own CU alone, so more waves in it raise that CU's rate.
inline int waves_per_split(int64_t wgs, int num_splits, int64_t s_max, int base, int max_p,
                           int cus) {
  const int64_t n = wgs * num_splits;
  if (cus <= 0 || n <= 0 || num_splits <= 0) return base;
  const int64_t chunk = ((s_max + num_splits - 1) / num_splits + 31) & ~int64_t(31);
  const int64_t tiles = chunk / 16;
  int P = base;
  for (const int p : {8, 12, 16})
    if (p <= max_p && n * p <= (int64_t)cus * 4 && tiles >= 2 * p) P = p;
  return P;
}

// Groups of at most 4 q-heads take the matrix-core scan instead of the VALU
// scan when the grid (one workgroup per request, kv-head and split) leaves
// CUs idle and the splits are short (at most kShortSplit tokens): such a
// launch is bound by each wave's chain of tiles, not by HBM, and the
// matrix-core scan's chain is shorter. Measured on MI355X (32Q/8KV, B = 1..8)
// against the VALU scan: 8-25 % faster at 64-512-token splits, 0-7 % at 1024,
// 4-20 % slower at 2048-4096 and 11-36 % slower at 8192-32768, where the
// VALU scan keeps more bytes in flight per CU. Full grids keep the VALU scan,
// which streams ~5 % faster there.
#ifndef GQA_MFMA_UNDERFILLED
#define GQA_MFMA_UNDERFILLED 1
#endif
constexpr int64_t kShortSplit = 1024;
inline bool use_mfma_underfilled(int B, int Hkv, int num_splits, int64_t s_max, int num_cus) {
  if (!GQA_MFMA_UNDERFILLED || num_cus <= 0 || num_splits <= 0) return false;
  const int64_t chunk = ((s_max + num_splits - 1) / num_splits + 31) & ~int64_t(31);
  return (int64_t)B * Hkv * num_splits < num_cus && chunk <= kShortSplit;
}

// MFMA scan: QK^T and PV on v_mfma_f32_16x16x32_bf16, up to 16 q-heads of a
// GQA group per wave. Launches one kernel: the slot-group layout over grid
// (num_splits, B) where use_mfma_slot says so, else over grid
// (Hkv * ceil(G/16), B, num_splits); returns the launch status.
hipError_t launch_scan_mfma(const ScanArgs& a, int B, hipStream_t stream);

}  // namespace gqa
