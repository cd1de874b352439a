// lane_probe.hip -- the cross-lane rules tests/c/chain_model.cpp assumes,
// measured on the GPU (one wave, in-bounds): a shuffle (ds_bpermute) from an
// inactive source lane returns 0, readlane reads an inactive lane's value, and
// a ballot sees only the active lanes.  Prints one line per rule; run by
// tests/test_gpu_lane_rules.py.
#include <hip/hip_runtime.h>
#include <cstdio>

__global__ void probe(int *shfl_div, int *shfl_full, int *readl, unsigned long long *bal) {
  const int lane = threadIdx.x;
  const int v = lane + 100;
  int r = -1;
  if (lane < 32) r = __shfl(v, lane + 32, 64); // sources 32..63 inactive here
  shfl_div[lane] = r;
  shfl_full[lane] = __shfl(v, (lane + 32) & 63, 64);
  int q = -1;
  if (lane < 32) q = __builtin_amdgcn_readlane(v, 40); // lane 40 inactive here
  readl[lane] = q;
  unsigned long long b = 0;
  if (lane < 32) b = __ballot(true);
  if (lane == 0) bal[0] = b;
}

int main() {
  int *a, *b, *c;
  unsigned long long *d;
  if (hipMalloc(&a, 256) != hipSuccess || hipMalloc(&b, 256) != hipSuccess ||
      hipMalloc(&c, 256) != hipSuccess || hipMalloc(&d, 8) != hipSuccess) {
    std::printf("hipMalloc failed\n");
    return 1;
  }
  probe<<<1, 64>>>(a, b, c, d);
  if (hipDeviceSynchronize() != hipSuccess) {
    std::printf("launch failed\n");
    return 1;
  }
  int ha[64], hb[64], hc[64];
  unsigned long long hd = 0;
  if (hipMemcpy(ha, a, 256, hipMemcpyDeviceToHost) != hipSuccess ||
      hipMemcpy(hb, b, 256, hipMemcpyDeviceToHost) != hipSuccess ||
      hipMemcpy(hc, c, 256, hipMemcpyDeviceToHost) != hipSuccess ||
      hipMemcpy(&hd, d, 8, hipMemcpyDeviceToHost) != hipSuccess) {
    std::printf("copy failed\n");
    return 1;
  }
  std::printf("shfl_inactive_source");
  for (int i = 0; i < 32; ++i) std::printf(" %d", ha[i]);
  std::printf("\nshfl_full_mask");
  for (int i = 0; i < 32; ++i) std::printf(" %d", hb[i]);
  std::printf("\nreadlane_inactive");
  for (int i = 0; i < 32; ++i) std::printf(" %d", hc[i]);
  std::printf("\nballot_half 0x%llx\n", hd);
  return 0;
}
