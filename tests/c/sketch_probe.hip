// sketch_probe -- replays item streams through the forms of the wave64
// space-saving update at capacity 128 (WaveSketch<4> in
// chunkedgreedy_amd/csrc/sketch.hpp, and one alternative kept here) and
// reports their cost and whether they agree.
//
//   sketch_probe ITEMS WAVES [HOT COLD PHOT]
//   sketch_probe 0 WAVES file PATH
//
// Each of WAVES waves (64 lanes) feeds its own stream of ITEMS items, 64 at a
// time as a full lane mask: a key drawn from HOT hot keys with probability
// PHOT, else from COLD cold keys, and the key's fixed weight 2/(1000 + d),
// d in [0, 100) (the form of csg's alpha = 2/(|r| + |s|)).  With `file`, every
// wave replays the stream in PATH instead: (int32 key, float32 weight) pairs,
// a multiple of 64 of them, as tests/c/hub_stream.py writes one row's stream.
// Forms:
//   0  add() item by item (the chunk tiers' loop for other capacities),
//   1  feed_generic() (the compiled two-loop update),
//   2  feed4() (the GCN-assembly update used at capacity 128),
//   3  RankSketch below (compiled): a rank per slot, the victim found by
//      ballot(rank == 0) instead of the DPP minimum; measured, not used.
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

namespace {

// Space-saving at capacity 128 that keeps each slot's rank in the eviction
// order (weight bits, 64j + p) -- cell j of physical lane p, the tie order of
// WaveSketch<4> -- so that the victim is the slot of rank 0.  The fill phase
// is feed_generic's; the ranks are built once when the sketch is full.  A
// weight change of slot h from key O to key N (O < N) lowers by one the rank
// of every slot X with O < X < N, and h's new rank is the number of slots
// below N.  Same slots as the other forms, item for item.
struct RankSketch {
  WaveSketch<4> s;
  uint32_t rank[2];
  bool ranked;

  __device__ __forceinline__ void clear() {
    s.clear();
    rank[0] = rank[1] = 0;
    ranked = false;
  }

  __device__ __forceinline__ void build_ranks() {
    const uint32_t lane = static_cast<uint32_t>(lane_id());
    const uint32_t w0 = __float_as_uint(s.wt[0]), w1 = __float_as_uint(s.wt[1]);
    uint32_t r0 = 0, r1 = 0;
    for (uint32_t q = 0; q < kWave; ++q) {
      const uint32_t a = static_cast<uint32_t>(readlane(__float_as_int(s.wt[0]), q));
      const uint32_t b = static_cast<uint32_t>(readlane(__float_as_int(s.wt[1]), q));
      r0 += (a < w0 || (a == w0 && q < lane)) + (b < w0);
      r1 += (a < w1 || (a == w1 && q < 64 + lane)) + (b < w1 || (b == w1 && q < lane));
    }
    rank[0] = r0;
    rank[1] = r1;
    ranked = true;
  }

  // Slot (jh, ph), of old rank rold, now holds weight wnew.
  __device__ __forceinline__ void rerank(int jh, int ph, uint32_t rold, float wnew) {
    const uint32_t lane = static_cast<uint32_t>(lane_id());
    const uint32_t wn = __float_as_uint(wnew);
    const uint32_t posh = 64u * static_cast<uint32_t>(jh) + static_cast<uint32_t>(ph);
    const uint32_t w0 = __float_as_uint(s.wt[0]), w1 = __float_as_uint(s.wt[1]);
    const bool l0 = w0 < wn || (w0 == wn && lane < posh);
    const bool l1 = w1 < wn || (w1 == wn && 64 + lane < posh);
    const uint32_t rn = __builtin_popcountll(ballot(l0)) + __builtin_popcountll(ballot(l1));
    if (l0 && rank[0] > rold) rank[0] -= 1;
    if (l1 && rank[1] > rold) rank[1] -= 1;
    if (lane == static_cast<uint32_t>(ph)) {
      if (jh == 0) rank[0] = rn;
      else rank[1] = rn;
    }
  }

  __device__ __forceinline__ void feed(uint64_t mask, int32_t other, float alpha) {
    const uint32_t lane = static_cast<uint32_t>(lane_id());
    while (mask != 0 && s.filled < 128) {
      const int i = __builtin_ctzll(mask);
      mask &= mask - 1;
      const int32_t k = readlane(other, i);
      const float w = readlane_f(alpha, i);
      if (s.hit_update<true>(k, w)) continue;
      const uint32_t f = static_cast<uint32_t>(s.filled);
      const uint32_t L = f / 4, c = f - L * 4;
      const uint64_t bit = 1ull << (L + 32u * (c & 1u));
      for (int j = 0; j < 2; ++j) {
        const uint64_t sel = (static_cast<uint32_t>(j) == (c >> 1)) ? bit : 0;
        s.key[j] = mask_select(sel, k, s.key[j]);
        s.wt[j] = __int_as_float(mask_select(sel, __float_as_int(w), __float_as_int(s.wt[j])));
      }
      s.filled += 1;
    }
    if (mask == 0) return;
    if (!ranked) build_ranks();
    while (mask != 0) {
      const int i = __builtin_ctzll(mask);
      mask &= mask - 1;
      const int32_t k = readlane(other, i);
      const float w = readlane_f(alpha, i);
      const uint64_t h0 = ballot(s.key[0] == k), h1 = ballot(s.key[1] == k);
      if ((h0 | h1) != 0) {
        const int jh = h0 != 0 ? 0 : 1;
        const int ph = __builtin_ctzll(h0 | h1);
        const float wo = readlane_f(jh == 0 ? s.wt[0] : s.wt[1], ph);
        const uint32_t rold =
            static_cast<uint32_t>(readlane(static_cast<int32_t>(jh == 0 ? rank[0] : rank[1]), ph));
        if (__builtin_amdgcn_inverse_ballot_w64(h0)) s.wt[0] = s.wt[0] + w;
        if (__builtin_amdgcn_inverse_ballot_w64(h1)) s.wt[1] = s.wt[1] + w;
        rerank(jh, ph, rold, wo + w);
        continue;
      }
      const uint64_t m0 = ballot(rank[0] == 0);
      const int jv = m0 != 0 ? 0 : 1;
      const uint64_t m = m0 != 0 ? m0 : ballot(rank[1] == 0);
      const int pv = __builtin_ctzll(m);
      const float wn = readlane_f(jv == 0 ? s.wt[0] : s.wt[1], pv) + w;
      if (lane == static_cast<uint32_t>(pv)) {
        if (jv == 0) {
          s.key[0] = k;
          s.wt[0] = wn;
        } else {
          s.key[1] = k;
          s.wt[1] = wn;
        }
      }
      rerank(jv, pv, 0u, wn);
    }
  }
};

} // namespace

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
  RankSketch rs;
  rs.clear();
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
    } else if constexpr (FORM == 2) {
      st.feed4(mask, o, a);
    } else {
      rs.feed(mask, o, a);
    }
    o = o_next;
    a = a_next;
  }
  const long long t1 = clock64();
  if constexpr (FORM == 3) st = rs.s;
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
    std::fprintf(stderr, "usage: %s ITEMS WAVES [HOT COLD PHOT] | 0 WAVES file PATH\n", argv[0]);
    return 1;
  }
  int n_items = std::atoi(argv[1]);
  const int waves = std::atoi(argv[2]);
  // (key, weight bits) pairs of a stream file, when one is named.
  std::vector<int32_t> fbuf;
  const bool from_file = argc > 4 && std::strcmp(argv[3], "file") == 0;
  if (from_file) {
    FILE *fp = std::fopen(argv[4], "rb");
    if (fp == nullptr) {
      std::fprintf(stderr, "cannot open %s\n", argv[4]);
      return 1;
    }
    int32_t pr[2];
    while (std::fread(pr, 4, 2, fp) == 2) {
      fbuf.push_back(pr[0]);
      fbuf.push_back(pr[1]);
    }
    std::fclose(fp);
    n_items = static_cast<int>(fbuf.size() / 2);
  }
  const int hot = (!from_file && argc > 3) ? std::atoi(argv[3]) : 100;
  const int cold = (!from_file && argc > 4) ? std::atoi(argv[4]) : 1000;
  const double phot = (!from_file && argc > 5) ? std::atof(argv[5]) : 0.5;
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
    if (from_file) {
      const size_t j = i % static_cast<size_t>(n_items);
      keys[i] = fbuf[2 * j];
      std::memcpy(&al[i], &fbuf[2 * j + 1], 4);
    }
  }
  constexpr int kForms = 4;
  int32_t *dk, *ok[kForms];
  float *da, *ow[kForms];
  long long *cy;
  CK(hipMalloc(&dk, N * 4));
  CK(hipMalloc(&da, N * 4));
  CK(hipMalloc(&cy, static_cast<size_t>(waves) * 8));
  for (int v = 0; v < kForms; ++v) {
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
  for (int v = 0; v < kForms; ++v) {
    float ms = 0.0f;
    for (int rep = 0; rep < 3; ++rep) {
      CK(hipEventRecord(e0));
      if (v == 0) probe<0><<<blocks, threads>>>(dk, da, n_items, ok[v], ow[v], cy);
      if (v == 1) probe<1><<<blocks, threads>>>(dk, da, n_items, ok[v], ow[v], cy);
      if (v == 2) probe<2><<<blocks, threads>>>(dk, da, n_items, ok[v], ow[v], cy);
      if (v == 3) probe<3><<<blocks, threads>>>(dk, da, n_items, ok[v], ow[v], cy);
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
  for (int v = 1; v < kForms; ++v) {
    CK(hipMemcpy(k1.data(), ok[v], S * 4, hipMemcpyDeviceToHost));
    CK(hipMemcpy(w1.data(), ow[v], S * 4, hipMemcpyDeviceToHost));
    const bool same = k0 == k1 && std::memcmp(w0.data(), w1.data(), S * 4) == 0;
    std::printf("form=%d equals_form0=%s\n", v, same ? "yes" : "no");
    all = all && same;
  }
  return all ? 0 : 2;
}
