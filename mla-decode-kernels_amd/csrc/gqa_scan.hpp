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

// MFMA scan: QK^T and PV on v_mfma_f32_16x16x32_bf16, up to 16 q-heads of a
// GQA group per wave. Launches one kernel: the slot-group layout over grid
// (num_splits, B) where use_mfma_slot says so, else over grid
// (Hkv * ceil(G/16), B, num_splits); returns the launch status.
hipError_t launch_scan_mfma(const ScanArgs& a, int B, hipStream_t stream);

}  // namespace gqa
