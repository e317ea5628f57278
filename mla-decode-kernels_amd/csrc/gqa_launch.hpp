// Host-side argument checks shared by the C-ABI launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace gqa {

// The checks python/gqa_decode_ext.cpp:16-62 makes on tensor shapes, restated
// for raw pointers and sizes, plus the limits of this build's launch geometry
// (batch in grid.y, 32-bit offsets inside one cache block). B == 0 is valid
// and launches nothing.
inline hipError_t check_common(const void* q, const void* k_cache, const void* v_cache,
                               const void* block_table, const void* seq_lens, const void* out,
                               int B, int Hq, int Hkv, int block_size, int max_blocks) {
  if (B < 0 || B > 65535) return hipErrorInvalidValue;
  if (Hq < 1 || Hkv < 1 || Hq % Hkv != 0) return hipErrorInvalidValue;
  if (block_size < 1 || max_blocks < 1) return hipErrorInvalidValue;
  // One block's K (or V) rows must be addressable with 32-bit element offsets.
  if ((int64_t)block_size * Hkv * 128 >= (int64_t(1) << 31)) return hipErrorInvalidValue;
  if ((int64_t)B * Hq > (int64_t(1) << 30)) return hipErrorInvalidValue;
  if (B > 0 && (!q || !k_cache || !v_cache || !block_table || !seq_lens || !out))
    return hipErrorInvalidValue;
  return hipSuccess;
}

// CU count of the current device, queried once per device (a racing first
// query stores the same value); 0 if it cannot be queried.
inline int device_cu_count() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  int cus = dev >= 0 && dev < 64 ? cached[dev].load(std::memory_order_relaxed) : 0;
  if (cus > 0) return cus;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    return 0;
  if (dev >= 0 && dev < 64) cached[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

}  // namespace gqa
