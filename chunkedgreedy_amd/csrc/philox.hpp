// philox.hpp -- Philox4x32-10 counter-based generator (Salmon, Moraes, Dror,
// Shaw, "Parallel random numbers: as easy as 1, 2, 3", SC'11): ten rounds of
// two 32x32->64 multiplies (0xD2511F53, 0xCD9E8D57) with the key bumped by
// the Weyl constants (0x9E3779B9, 0xBB67AE85) after each round.  Checked on
// the GPU against the published known-answer vectors by
// tests/test_gpu_philox.py.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sporder_hip {

__device__ __forceinline__ uint4 philox4x32_10(uint4 ctr, uint2 key) {
  const uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u;
  const uint32_t W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint32_t hi0 = __umulhi(M0, ctr.x), lo0 = M0 * ctr.x;
    const uint32_t hi1 = __umulhi(M1, ctr.z), lo1 = M1 * ctr.z;
    ctr = make_uint4(hi1 ^ ctr.y ^ key.x, lo1, hi0 ^ ctr.w ^ key.y, lo0);
    key.x += W0;
    key.y += W1;
  }
  return ctr;
}

} // namespace sporder_hip
