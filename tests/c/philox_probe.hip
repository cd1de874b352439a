// philox_probe.hip -- the library's Philox4x32-10 (chunkedgreedy_amd/csrc/
// philox.hpp) on the GPU for three counter/key pairs; prints one line of four
// hex words each.  Run by tests/test_gpu_philox.py.
#include "../../chunkedgreedy_amd/csrc/philox.hpp"

#include <cstdio>

__global__ void kat(uint4 *out) {
  const uint4 ctr[3] = {make_uint4(0u, 0u, 0u, 0u),
                        make_uint4(0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu),
                        make_uint4(0x243f6a88u, 0x85a308d3u, 0x13198a2eu, 0x03707344u)};
  const uint2 key[3] = {make_uint2(0u, 0u), make_uint2(0xffffffffu, 0xffffffffu),
                        make_uint2(0xa4093822u, 0x299f31d0u)};
  const int i = threadIdx.x;
  if (i < 3) out[i] = sporder_hip::philox4x32_10(ctr[i], key[i]);
}

int main() {
  uint4 *d = nullptr;
  if (hipMalloc(&d, 3 * sizeof(uint4)) != hipSuccess) return 1;
  kat<<<1, 64>>>(d);
  uint4 h[3];
  if (hipDeviceSynchronize() != hipSuccess ||
      hipMemcpy(h, d, sizeof(h), hipMemcpyDeviceToHost) != hipSuccess) {
    std::printf("failed\n");
    return 1;
  }
  for (int i = 0; i < 3; ++i) std::printf("%08x %08x %08x %08x\n", h[i].x, h[i].y, h[i].z, h[i].w);
  return 0;
}
