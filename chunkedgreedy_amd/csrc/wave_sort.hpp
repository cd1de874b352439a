// wave_sort.hpp -- one wave sorting a u32 array in LDS (bitonic network).
#pragma once

#include "common.hpp"

namespace sporder_hip {

__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// Ascending sort of a[0, size) in LDS by one wave: bitonic network in the
// "mirror" form (first stage of each merge compares i with its mirror in the
// block, later stages are half-cleaners), in which every exchange is
// ascending, so positions >= size act as +infinity and are never touched.
__device__ inline void wave_sort_lds(uint32_t *a, int32_t size) {
  const int lane = lane_id();
  int32_t p2 = 1;
  while (p2 < size) p2 <<= 1;
  for (int32_t kk = 2; kk <= p2; kk <<= 1) {
    for (int32_t j = kk >> 1; j > 0; j >>= 1) {
      for (int32_t t = lane; t < (p2 >> 1); t += kWave) {
        const int32_t lo = ((t & ~(j - 1)) << 1) | (t & (j - 1));
        // First stage of the level: partner is the mirror inside the block.
        const int32_t hi = (j == (kk >> 1)) ? (lo | (kk - 1)) - (lo & (kk - 1)) : lo + j;
        if (hi < size) {
          const uint32_t x = a[lo], y = a[hi];
          if (x > y) {
            a[lo] = y;
            a[hi] = x;
          }
        }
      }
      wave_lds_fence();
    }
  }
}

} // namespace sporder_hip
