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
//      ballot(rank == 0) instead of the DPP minimum; measured, not used,
//   4  QueueSketch below: feed4() with the eviction order kept between
//      evictions (a sort serves about 60 evictions on C3's hub stream, the
//      front taken by scalar tests); measured, not used.
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

// The eviction order of a full capacity-128 sketch (WaveSketch<4>), kept
// between evictions by QueueSketch::feed().  One bitonic sort of the 128 (weight, 64j + p)
// keys puts the 64 smallest slots, in eviction order, one per lane; later
// evictions take them from the front while the front's weight is below
// `bound`, a lower bound of every slot outside the unevicted queue: the
// 65th smallest weight at the sort, lowered to each evicted slot's new
// weight.  A hit on a queued slot takes it out of the queue and lowers the
// bound to its new weight.  Queued slots are untouched and stay in key order,
// and every other slot weighs at least the bound, so a front below the bound
// is the minimum key that the full reduction would find; otherwise the
// eviction sorts again.
struct MinQueue {
  uint32_t qw;    // lane r: weight bits of the r-th smallest slot at the sort
  uint32_t qs;    // lane r: that slot as 64j + p (local cell j, physical lane p)
  int32_t head;   // wave-uniform: next lane to evict; 64 = nothing queued
  uint32_t bound; // wave-uniform: see above; 0 = sort at the next eviction
  uint64_t qm[2]; // wave-uniform, per cell: lanes whose slot is queued, not evicted

  __device__ __forceinline__ void reset() {
    qw = 0;
    qs = 0;
    head = 64;
    bound = 0;
    qm[0] = 0;
    qm[1] = 0;
  }
};

// Form 4: WaveSketch<4> with its eviction order kept in a MinQueue.
struct QueueSketch {
  WaveSketch<4> s;
  MinQueue q;

  __device__ __forceinline__ void clear() {
    s.clear();
    q.reset();
  }

  // feed4() on a full sketch with the eviction order kept in a
  // MinQueue: the same updates item by item, but an eviction takes the
  // queue's front (two lane reads and scalar tests) instead of the wave
  // minimum (six DPP steps and two vector-to-scalar round trips), and sorts
  // the sketch again only when the front may no longer be the minimum.  On
  // one hub row's long stream the new weight (minimum + w) lands above the
  // queue's remaining slots nearly always, so each sort serves about 60
  // evictions.  While slots are free it is feed4(), and the queue is empty.
  __device__ __forceinline__ void feed(uint64_t mask, int32_t other, float alpha) {
        if (__builtin_amdgcn_readfirstlane(s.filled) < 128) {
      s.feed4(mask, other, alpha);
      q.reset();
      return;
    }
    const int lane = lane_id();
    mask = uniform_mask(mask);
    for (;;) {
      uint32_t need, kk, ww;
      queue_steps(mask, other, alpha, need, kk, ww);
      if (need == 0) return;
      // The front may not be the minimum: sort the 128 (weight, 64j + p)
      // keys, queue the 64 smallest, and evict the smallest for (kk, ww).
      uint32_t hi[2] = {__float_as_uint(s.wt[0]), __float_as_uint(s.wt[1])};
      uint32_t lo[2] = {static_cast<uint32_t>(lane), static_cast<uint32_t>(64 + lane)};
      bitonic_sort128(hi, lo);
      const uint64_t kth =
          (static_cast<uint64_t>(static_cast<uint32_t>(readlane(static_cast<int32_t>(hi[0]), 63)))
           << 32) |
          static_cast<uint32_t>(readlane(static_cast<int32_t>(lo[0]), 63));
      const uint64_t mine0 = (static_cast<uint64_t>(__float_as_uint(s.wt[0])) << 32) |
                             static_cast<uint32_t>(lane);
      const uint64_t mine1 = (static_cast<uint64_t>(__float_as_uint(s.wt[1])) << 32) |
                             static_cast<uint32_t>(64 + lane);
      uint64_t qm0 = ballot(mine0 <= kth), qm1 = ballot(mine1 <= kth);
      const uint32_t wq = static_cast<uint32_t>(readlane(static_cast<int32_t>(hi[0]), 0));
      const uint32_t slot = static_cast<uint32_t>(readlane(static_cast<int32_t>(lo[0]), 0));
      uint32_t bound = static_cast<uint32_t>(readlane(static_cast<int32_t>(hi[1]), 0));
      q.qw = hi[0];
      q.qs = lo[0];
      const float wn = __uint_as_float(ww) + __uint_as_float(wq); // the slot holds wq
      const uint64_t sel = 1ull << (slot & 63u);
      if (slot < 64u) {
        s.key[0] = mask_select(sel, static_cast<int32_t>(kk), s.key[0]);
        s.wt[0] = __int_as_float(mask_select(sel, __float_as_int(wn), __float_as_int(s.wt[0])));
        qm0 &= ~sel;
      } else {
        s.key[1] = mask_select(sel, static_cast<int32_t>(kk), s.key[1]);
        s.wt[1] = __int_as_float(mask_select(sel, __float_as_int(wn), __float_as_int(s.wt[1])));
        qm1 &= ~sel;
      }
      bound = min(bound, __float_as_uint(wn));
      q.bound = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int32_t>(bound)));
      q.qm[0] = uniform_mask(qm0);
      q.qm[1] = uniform_mask(qm1);
      q.head = 1;
      if (mask == 0) return;
    }
  }

  static __device__ __forceinline__ uint64_t uniform_mask(uint64_t m) {
    return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int32_t>(m))) |
           (static_cast<uint64_t>(static_cast<uint32_t>(
                __builtin_amdgcn_readfirstlane(static_cast<int32_t>(m >> 32))))
            << 32);
  }

  // feed()'s item loop, one block of GCN assembly in feed4()'s style.  A
  // hit adds w in both cells by their hit masks; when it hits a queued slot,
  // that slot leaves the queue (its mask bit cleared) and the bound drops to
  // its new weight (v_readlane of the hit lane).  A miss skips front entries
  // whose slot left the queue, and evicts the front when its weight is below
  // the bound: v_writelane of k at the slot's lane (M0), wq + w by a select
  // on the one-hot lane mask, the slot's queue bit cleared, the bound
  // lowered to the new weight.  Otherwise it stops with need = 1 and the
  // item (kk, ww) for the caller to evict after a sort; need = 0 when the
  // mask is exhausted.  Every lane of the wave must be active.
  __device__ __forceinline__ void queue_steps(uint64_t &mask, int32_t other, float alpha, uint32_t &need,
                                              uint32_t &kk, uint32_t &ww) {
    uint32_t i, p, slot, wq, nw, m0_saved;
    uint64_t h0, h1, any, sel;
    float t;
    int32_t head = __builtin_amdgcn_readfirstlane(q.head);
    uint32_t bound = static_cast<uint32_t>(
        __builtin_amdgcn_readfirstlane(static_cast<int32_t>(q.bound)));
    uint64_t qm0 = uniform_mask(q.qm[0]), qm1 = uniform_mask(q.qm[1]);
    asm volatile(
        "s_mov_b32 %[m0s], m0\n\t"
        "s_mov_b32 %[need], 0\n\t"
        "s_cmp_eq_u64 %[mask], 0\n\t"
        "s_cbranch_scc1 9f\n"
        "5:\n\t"
        "s_ff1_i32_b64 %[i], %[mask]\n\t"
        "s_bitset0_b64 %[mask], %[i]\n\t"
        "v_readlane_b32 %[kk], %[other], %[i]\n\t"
        "v_readlane_b32 %[ww], %[alpha], %[i]\n\t"
        "s_nop 0\n\t"
        "v_cmp_eq_u32_e64 %[h0], %[kk], %[k0]\n\t"
        "v_cmp_eq_u32_e64 %[h1], %[kk], %[k1]\n\t"
        "s_or_b64 %[any], %[h0], %[h1]\n\t"
        "s_cbranch_scc0 6f\n\t"
        // hit
        "v_add_f32_e64 %[t], %[ww], %[w0]\n\t"
        "v_cndmask_b32_e64 %[w0], %[w0], %[t], %[h0]\n\t"
        "v_add_f32_e64 %[t], %[ww], %[w1]\n\t"
        "v_cndmask_b32_e64 %[w1], %[w1], %[t], %[h1]\n\t"
        "s_and_b64 %[h0], %[h0], %[qm0]\n\t"
        "s_and_b64 %[h1], %[h1], %[qm1]\n\t"
        "s_or_b64 %[any], %[h0], %[h1]\n\t"
        "s_cbranch_scc1 8f\n\t"
        "s_cmp_lg_u64 %[mask], 0\n\t"
        "s_cbranch_scc1 5b\n\t"
        "s_branch 9f\n"
        // the hit slot was queued: it leaves the queue
        "8:\n\t"
        "s_andn2_b64 %[qm0], %[qm0], %[h0]\n\t"
        "s_andn2_b64 %[qm1], %[qm1], %[h1]\n\t"
        "s_cmp_eq_u64 %[h0], 0\n\t"
        "s_cbranch_scc1 81f\n\t"
        "s_ff1_i32_b64 %[p], %[h0]\n\t"
        "v_readlane_b32 %[nw], %[w0], %[p]\n\t"
        "s_branch 82f\n"
        "81:\n\t"
        "s_ff1_i32_b64 %[p], %[h1]\n\t"
        "v_readlane_b32 %[nw], %[w1], %[p]\n"
        "82:\n\t"
        "s_min_u32 %[bound], %[bound], %[nw]\n\t"
        "s_cmp_lg_u64 %[mask], 0\n\t"
        "s_cbranch_scc1 5b\n\t"
        "s_branch 9f\n"
        // miss: the queue's front, past the slots that left it
        "6:\n\t"
        "s_cmp_ge_u32 %[head], 64\n\t"
        "s_cbranch_scc1 7f\n\t"
        "v_readlane_b32 %[slot], %[qs], %[head]\n\t"
        "v_readlane_b32 %[wq], %[qw], %[head]\n\t"
        "s_and_b32 %[p], %[slot], 63\n\t"
        "s_cmp_ge_u32 %[slot], 64\n\t"
        "s_cselect_b64 %[sel], %[qm1], %[qm0]\n\t"
        "s_bitcmp1_b64 %[sel], %[p]\n\t"
        "s_cbranch_scc1 61f\n\t"
        "s_add_u32 %[head], %[head], 1\n\t"
        "s_branch 6b\n"
        "61:\n\t"
        "s_cmp_lt_u32 %[wq], %[bound]\n\t"
        "s_cbranch_scc0 7f\n\t"
        "s_add_u32 %[head], %[head], 1\n\t"
        "s_lshl_b64 %[sel], 1, %[p]\n\t"
        "s_mov_b32 m0, %[p]\n\t"
        "s_cmp_ge_u32 %[slot], 64\n\t"
        "s_cbranch_scc1 65f\n\t"
        "s_andn2_b64 %[qm0], %[qm0], %[sel]\n\t"
        "v_writelane_b32 %[k0], %[kk], m0\n\t"
        "v_add_f32_e64 %[t], %[ww], %[w0]\n\t"
        "v_cndmask_b32_e64 %[w0], %[w0], %[t], %[sel]\n\t"
        "s_branch 66f\n"
        "65:\n\t"
        "s_andn2_b64 %[qm1], %[qm1], %[sel]\n\t"
        "v_writelane_b32 %[k1], %[kk], m0\n\t"
        "v_add_f32_e64 %[t], %[ww], %[w1]\n\t"
        "v_cndmask_b32_e64 %[w1], %[w1], %[t], %[sel]\n"
        "66:\n\t"
        "s_nop 0\n\t"
        "v_readlane_b32 %[nw], %[t], %[p]\n\t"
        "s_min_u32 %[bound], %[bound], %[nw]\n\t"
        "s_cmp_lg_u64 %[mask], 0\n\t"
        "s_cbranch_scc1 5b\n\t"
        "s_branch 9f\n"
        "7:\n\t"
        "s_mov_b32 %[need], 1\n"
        "9:\n\t"
        "s_mov_b32 m0, %[m0s]"
        : [k0] "+v"(s.key[0]), [k1] "+v"(s.key[1]), [w0] "+v"(s.wt[0]), [w1] "+v"(s.wt[1]),
          [mask] "+s"(mask), [head] "+s"(head), [bound] "+s"(bound), [qm0] "+s"(qm0),
          [qm1] "+s"(qm1), [need] "=&s"(need), [kk] "=&s"(kk), [ww] "=&s"(ww), [t] "=&v"(t),
          [i] "=&s"(i), [p] "=&s"(p), [slot] "=&s"(slot), [wq] "=&s"(wq), [nw] "=&s"(nw),
          [h0] "=&s"(h0), [h1] "=&s"(h1), [any] "=&s"(any), [sel] "=&s"(sel),
          [m0s] "=&s"(m0_saved)
        : [other] "v"(other), [alpha] "v"(alpha), [qw] "v"(q.qw), [qs] "v"(q.qs)
        : "scc");
    q.head = head;
    q.bound = bound;
    q.qm[0] = qm0;
    q.qm[1] = qm1;
  }
};

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
  QueueSketch qsk;
  qsk.clear();
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
    } else if constexpr (FORM == 3) {
      rs.feed(mask, o, a);
    } else {
      qsk.feed(mask, o, a);
    }
    o = o_next;
    a = a_next;
  }
  const long long t1 = clock64();
  if constexpr (FORM == 3) st = rs.s;
  if constexpr (FORM == 4) st = qsk.s;
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
  constexpr int kForms = 5;
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
      if (v == 4) probe<4><<<blocks, threads>>>(dk, da, n_items, ok[v], ow[v], cy);
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
