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
};

// MFMA scan: QK^T and PV on v_mfma_f32_16x16x32_bf16, up to 16 q-heads of a
// GQA group per wave. Launches one kernel over grid
// (Hkv * ceil(G/16), B, num_splits); returns the launch status.
hipError_t launch_scan_mfma(const ScanArgs& a, int B, hipStream_t stream);

}  // namespace gqa
