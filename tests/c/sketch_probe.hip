// sketch_probe -- replays synthetic item streams through the three forms of
// the wave64 space-saving update in chunkedgreedy_amd/csrc/sketch.hpp at
// capacity 128 (WaveSketch<4>) and reports their cost and whether they agree.
//
//   sketch_probe ITEMS WAVES [HOT COLD PHOT]
//
// Each of WAVES waves (64 lanes) feeds its own stream of ITEMS items, 64 at a
// time as a full lane mask: a key drawn from HOT hot keys with probability
// PHOT, else from COLD cold keys, and the key's fixed weight 2/(1000 + d),
// d in [0, 100) (the form of csg's alpha = 2/(|r| + |s|)).  Forms:
//   0  add() item by item (the chunk tiers' loop for other capacities),
//   1  feed_generic() (the compiled two-loop update),
//   2  feed4() (the GCN-assembly update used at capacity 128).
// Per form: kernel time (third of three launches), whole-GPU items/s, and
// the mean s_memtime cycles per item of a wave.  Then whether each form's
// final slots (keys and weight bits) equal form 0's.  Exit status 0 when they
// do, 2 when not.  One wave gives the latency of one long stream (C3's hub
// row); 4096 or 8192 waves give the throughput at four or eight waves per
// SIMD (C5's tiers).
#include "sketch.hpp"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

using namespace sporder_hip;

template <int FORM>
__global__ void __launch_bounds__(256)
    probe(const int32_t *__restrict__ keys, const float *__restrict__ alphas, int n_items,
          int32_t *__restrict__ out_key, float *__restrict__ out_wt,
          long long *__restrict__ cycles) {
  const int lane = lane_id();
  const int w = (blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const int32_t *K = keys + static_cast<size_t>(w) * n_items;
  const float *A = alphas + static_cast<size_t>(w) * n_items;
  WaveSketch<4> st;
  st.clear();
  int32_t o = K[lane];
  float a = A[lane];
  const long long t0 = clock64();
  for (int b = 0; b < n_items; b += kWave) {
    // The next batch's load in flight while this one is applied.
    const int32_t o_next = b + kWave < n_items ? K[b + kWave + lane] : 0;
    const float a_next = b + kWave < n_items ? A[b + kWave + lane] : 0.0f;
    const uint64_t mask = ballot(true);
    if constexpr (FORM == 0) {
      uint64_t m = mask;
      while (m) {
        const int i = __builtin_ctzll(m);
        st.add(readlane(o, i), readlane_f(a, i));
        m = clear_bit(m, i);
      }
    } else if constexpr (FORM == 1) {
      st.feed_generic(mask, o, a);
    } else {
      st.feed4(mask, o, a);
    }
    o = o_next;
    a = a_next;
  }
  const long long t1 = clock64();
  const size_t base = static_cast<size_t>(w) * 128;
  out_key[base + lane] = st.key[0];
  out_key[base + kWave + lane] = st.key[1];
  out_wt[base + lane] = st.wt[0];
  out_wt[base + kWave + lane] = st.wt[1];
  if (lane == 0) cycles[w] = t1 - t0;
}

#define CK(x)                                                                 \
  do {                                                                        \
    hipError_t e_ = (x);                                                      \
    if (e_ != hipSuccess) {                                                   \
      std::fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), \
                   __LINE__);                                                 \
      return 1;                                                               \
    }                                                                         \
  } while (0)

int main(int argc, char **argv) {
  if (argc < 3) {
    std::fprintf(stderr, "usage: %s ITEMS WAVES [HOT COLD PHOT]\n", argv[0]);
    return 1;
  }
  const int n_items = std::atoi(argv[1]);
  const int waves = std::atoi(argv[2]);
  const int hot = argc > 3 ? std::atoi(argv[3]) : 100;
  const int cold = argc > 4 ? std::atoi(argv[4]) : 1000;
  const double phot = argc > 5 ? std::atof(argv[5]) : 0.5;
  if (n_items < kWave || n_items % kWave != 0 || waves < 1 || (waves > 4 && waves % 4 != 0) ||
      hot < 1 || cold < 1) {
    std::fprintf(stderr, "ITEMS must be a positive multiple of 64, WAVES 1..4 or a multiple of 4\n");
    return 1;
  }
  std::printf("items_per_wave=%d waves=%d hot=%d cold=%d phot=%.2f\n", n_items, waves, hot, cold,
              phot);
  const size_t N = static_cast<size_t>(n_items) * waves;
  std::vector<int32_t> keys(N);
  std::vector<float> al(N);
  std::mt19937_64 rng(12345);
  std::vector<float> alpha_of(static_cast<size_t>(hot + cold));
  for (auto &x : alpha_of) x = 2.0f / static_cast<float>(1000 + static_cast<int>(rng() % 100));
  for (size_t i = 0; i < N; ++i) {
    const double u = static_cast<double>(rng() >> 11) * (1.0 / 9007199254740992.0);
    const int s = u < phot ? static_cast<int>(rng() % hot) : hot + static_cast<int>(rng() % cold);
    keys[i] = s;
    al[i] = alpha_of[static_cast<size_t>(s)];
  }
  int32_t *dk, *ok[3];
  float *da, *ow[3];
  long long *cy;
  CK(hipMalloc(&dk, N * 4));
  CK(hipMalloc(&da, N * 4));
  CK(hipMalloc(&cy, static_cast<size_t>(waves) * 8));
  for (int v = 0; v < 3; ++v) {
    CK(hipMalloc(&ok[v], static_cast<size_t>(waves) * 128 * 4));
    CK(hipMalloc(&ow[v], static_cast<size_t>(waves) * 128 * 4));
  }
  CK(hipMemcpy(dk, keys.data(), N * 4, hipMemcpyHostToDevice));
  CK(hipMemcpy(da, al.data(), N * 4, hipMemcpyHostToDevice));
  const int threads = waves >= 4 ? 256 : kWave * waves;
  const int blocks = waves * kWave / threads;
  hipEvent_t e0, e1;
  CK(hipEventCreate(&e0));
  CK(hipEventCreate(&e1));
  std::vector<long long> hc(static_cast<size_t>(waves));
  for (int v = 0; v < 3; ++v) {
    float ms = 0.0f;
    for (int rep = 0; rep < 3; ++rep) {
      CK(hipEventRecord(e0));
      if (v == 0) probe<0><<<blocks, threads>>>(dk, da, n_items, ok[v], ow[v], cy);
      if (v == 1) probe<1><<<blocks, threads>>>(dk, da, n_items, ok[v], ow[v], cy);
      if (v == 2) probe<2><<<blocks, threads>>>(dk, da, n_items, ok[v], ow[v], cy);
      CK(hipGetLastError());
      CK(hipEventRecord(e1));
      CK(hipEventSynchronize(e1));
      CK(hipEventElapsedTime(&ms, e0, e1));
    }
    CK(hipMemcpy(hc.data(), cy, static_cast<size_t>(waves) * 8, hipMemcpyDeviceToHost));
    double mean = 0.0;
    for (long long c : hc) mean += static_cast<double>(c);
    mean /= waves;
    std::printf("form=%d ms=%.3f items_per_s=%.3e cycles_per_item=%.1f\n", v, ms,
                static_cast<double>(N) / (ms * 1e-3), mean / n_items);
  }
  const size_t S = static_cast<size_t>(waves) * 128;
  std::vector<int32_t> k0(S), k1(S);
  std::vector<float> w0(S), w1(S);
  CK(hipMemcpy(k0.data(), ok[0], S * 4, hipMemcpyDeviceToHost));
  CK(hipMemcpy(w0.data(), ow[0], S * 4, hipMemcpyDeviceToHost));
  bool all = true;
  for (int v = 1; v < 3; ++v) {
    CK(hipMemcpy(k1.data(), ok[v], S * 4, hipMemcpyDeviceToHost));
    CK(hipMemcpy(w1.data(), ow[v], S * 4, hipMemcpyDeviceToHost));
    const bool same = k0 == k1 && std::memcmp(w0.data(), w1.data(), S * 4) == 0;
    std::printf("form=%d equals_form0=%s\n", v, same ? "yes" : "no");
    all = all && same;
  }
  return all ? 0 : 2;
}
