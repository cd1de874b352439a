// csg.hip -- Chunked Greedy (sporder-csg): chunk-restricted space-saving
// sketch + top-k, the per-chunk greedy chain, table statistics and the C-ABI
// entry points sporder_chunk_similarity_greedy, sporder_similarity_graph and
// sporder_chunk_similarity_top_k.
//
// Semantics follow the reference bit for bit:
//   sketch stream  sporder/src/common/chunk_similarity_top_k.cu:30-88
//   space-saving   sporder/src/common/warp_spacesaving.cuh:12-151
//   arg-reductions sporder/src/common/cuda_util.cuh:66-87
//   greedy         sporder/src/csg/chunk_similarity_greedy.cu:14-98
//   stats          sporder/src/common/similarity_top_k.cu:120-172,
//                  sporder/src/csg/stats_collector.cu:43-63
//
// Mapping to gfx950 (wave64).  The reference's sketch lives in one 32-lane
// warp: logical lane L owns cells c = 0..CELLS-1 (M = 32*CELLS slots).  Here
// one wave64 serves one row and spreads the slots over all 64 lanes: physical
// lane p holds logical lane L = p & 31 and the cells c = 2j + (p >> 5),
// j = 0..ceil(CELLS/2)-1.  Every tie rule of the reference depends only on
// (L, c), so the arrangement is free:
//   - a new key goes to the first empty slot in order s = L*CELLS + c, which
//     is a wave-uniform counter instead of a find(-1) + ballot;
//   - eviction takes the minimum of (weight, c*32 + L), reduced over the
//     wave with a butterfly;
//   - top-k output merges the per-logical-lane selection-sorted lists with
//     ties to the smaller logical lane.
// The candidate stream of a row is gathered 64 entries at a time from the
// concatenation of its columns' CSC segments (a wave prefix sum over segment
// lengths finds each lane's segment), so a row's column walks are issued in
// parallel instead of one column after another; items are then applied in
// stream order.
#include "common.hpp"

#include <algorithm>
#include <chrono>

namespace sporder_hip {

namespace {

constexpr int kSketchBlock = 256;
constexpr int kSketchWaves = kSketchBlock / kWave;
// Column segments longer than this are trimmed to the chunk's row range by
// binary search before gathering (they are sorted by row).  Only entries the
// chunk filter rejects are skipped, so the stream is unchanged.
constexpr int kTrimLen = 64;

__device__ __forceinline__ int32_t lower_bound_dev(const int32_t *a, int32_t lo,
                                                   int32_t hi, int32_t t) {
  while (lo < hi) {
    int32_t mid = lo + (hi - lo) / 2;
    if (a[mid] < t) {
      lo = mid + 1;
    } else {
      hi = mid;
    }
  }
  return lo;
}

// Space-saving sketch of capacity 32*CELLS spread over one wave64.
template <int CELLS> struct WaveSketch {
  static constexpr int LC = (CELLS + 1) / 2; // cells held per physical lane
  static constexpr int M = 32 * CELLS;
  int32_t key[LC];
  float wt[LC];
  int32_t filled; // wave-uniform: slots taken so far (fill order L*CELLS+c)

  __device__ __forceinline__ void clear() {
#pragma unroll
    for (int j = 0; j < LC; ++j) {
      key[j] = -1;
      wt[j] = 0.0f;
    }
    filled = 0;
  }

  // Apply one item; k and w are wave-uniform.
  __device__ __forceinline__ void add(int32_t k, float w) {
    const int lane = lane_id();
    bool hit = false;
#pragma unroll
    for (int j = 0; j < LC; ++j) {
      if (key[j] == k) {
        wt[j] += w;
        hit = true;
      }
    }
    if (ballot(hit)) {
      return;
    }
    if (filled < M) {
      // Slot s = L*CELLS + c: logical lane L, cell c -> physical lane
      // L + 32*(c & 1), local cell c >> 1.
      int L = filled / CELLS, c = filled - L * CELLS;
      int owner = L + 32 * (c & 1), jj = c >> 1;
#pragma unroll
      for (int j = 0; j < LC; ++j) {
        if (lane == owner && j == jj) {
          key[j] = k;
          wt[j] = w;
        }
      }
      filled += 1;
      return;
    }
    // Evict argmin over slots of (weight, c*32 + L).
    const int L = lane & 31, h = lane >> 5;
    float best_w = __builtin_inff();
    int32_t best_k = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < LC; ++j) {
      int c = 2 * j + h;
      if (c < CELLS) {
        int32_t ck = (c << 5) | L;
        if (wt[j] < best_w || (wt[j] == best_w && ck < best_k)) {
          best_w = wt[j];
          best_k = ck;
        }
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      float ow = __shfl_xor(best_w, off, kWave);
      int32_t ok = __shfl_xor(best_k, off, kWave);
      if (ow < best_w || (ow == best_w && ok < best_k)) {
        best_w = ow;
        best_k = ok;
      }
    }
    int c = best_k >> 5;
    int owner = (best_k & 31) + 32 * (c & 1), jj = c >> 1;
#pragma unroll
    for (int j = 0; j < LC; ++j) {
      if (lane == owner && j == jj) {
        key[j] = k;
        wt[j] += w; // inherits the evicted weight
      }
    }
  }

  // Reference select_top_k: per-logical-lane selection sort (strict '>',
  // stop at -1), then up to k rounds emitting the head of the lane with the
  // largest head weight (ties -> smaller lane; exhausted lanes show 0.0f).
  // Writes all k entries of `out` (unused ones as the zero entry).
  __device__ __forceinline__ void select_top_k(int32_t k, uint64_t *out) {
    const int lane = lane_id();
    // Gather logical lane L's cells into physical lane L (< 32).
    int32_t fk[CELLS];
    float fw[CELLS];
#pragma unroll
    for (int j = 0; j < LC; ++j) {
      int32_t hk = __shfl(key[j], (lane & 31) + 32, kWave);
      float hw = __shfl(wt[j], (lane & 31) + 32, kWave);
      fk[2 * j] = key[j];
      fw[2 * j] = wt[j];
      if (2 * j + 1 < CELLS) {
        fk[2 * j + 1] = hk;
        fw[2 * j + 1] = hw;
      }
    }
    // Selection sort, literally as the reference (not stable).
#pragma unroll
    for (int i = 0; i < CELLS - 1; ++i) {
      if (fk[i] == -1) break;
      int best = i;
      float bw = fw[i];
#pragma unroll
      for (int j = i + 1; j < CELLS; ++j) {
        if (fk[j] == -1) break;
        if (fw[j] > bw) {
          best = j;
          bw = fw[j];
        }
      }
      if (best != i) {
        // Swap cells i and best (best is a run-time index: select by loop).
        int32_t tk = fk[i];
        float tw = fw[i];
#pragma unroll
        for (int j = i + 1; j < CELLS; ++j) {
          if (j == best) {
            fk[i] = fk[j];
            fw[i] = fw[j];
            fk[j] = tk;
            fw[j] = tw;
          }
        }
      }
    }
    // k-way merge; lane (i & 63) keeps output entry i in register i >> 6.
    uint64_t outv[4] = {0, 0, 0, 0};
    for (int32_t i = 0; i < k; ++i) {
      bool live = lane < 32 && fk[0] != -1;
      if (ballot(live) == 0) break;
      float v = lane < 32 ? fw[0] : -__builtin_inff();
      int32_t who = lane;
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) {
        float ov = __shfl_xor(v, off, kWave);
        int32_t ow = __shfl_xor(who, off, kWave);
        if (ov > v || (ov == v && ow < who)) {
          v = ov;
          who = ow;
        }
      }
      int winner = __builtin_amdgcn_readfirstlane(who);
      int32_t wk = readlane(fk[0], winner);
      float ww = readlane_f(fw[0], winner);
      int slot = i >> 6;
      if (lane == (i & 63)) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (r == slot) outv[r] = pack_wi(wk, ww);
        }
      }
      if (lane == winner) {
#pragma unroll
        for (int j = 0; j < CELLS - 1; ++j) {
          fk[j] = fk[j + 1];
          fw[j] = fw[j + 1];
        }
        fk[CELLS - 1] = -1;
        fw[CELLS - 1] = 0.0f;
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      int idx = r * 64 + lane;
      if (idx < k) out[idx] = outv[r];
    }
  }
};

// One wave per row (grid-stride).  Rows of length 0 get an all-zero table row.
template <int CELLS>
__global__ void __launch_bounds__(kSketchBlock)
    chunk_sketch_kernel(int32_t n, int32_t k, int32_t chunk_size,
                        const int32_t *__restrict__ row_ptr,
                        const int32_t *__restrict__ col_ind,
                        const int32_t *__restrict__ col_ptr,
                        const int32_t *__restrict__ row_ind,
                        uint64_t *__restrict__ table) {
  const int lane = lane_id();
  const int64_t wave0 =
      static_cast<int64_t>(blockIdx.x) * kSketchWaves + threadIdx.x / kWave;
  const int64_t nwaves = static_cast<int64_t>(gridDim.x) * kSketchWaves;
  WaveSketch<CELLS> store;

  for (int64_t row64 = wave0; row64 < n; row64 += nwaves) {
    const int32_t row = static_cast<int32_t>(row64);
    uint64_t *out = table + static_cast<size_t>(row) * k;
    const int32_t rs = row_ptr[row], re = row_ptr[row + 1];
    const int32_t row_size = re - rs;
    if (row_size == 0) {
      for (int32_t j = lane; j < k; j += kWave) out[j] = 0;
      continue;
    }
    const int32_t cs = (row / chunk_size) * chunk_size;
    int32_t ce = cs + chunk_size;
    if (ce > n || ce < cs) ce = n;

    store.clear();
    for (int32_t pb = rs; pb < re; pb += kWave) {
      const int32_t p = pb + lane;
      int32_t a = 0, b = 0;
      if (p < re) {
        int32_t col = col_ind[p];
        a = col_ptr[col];
        b = col_ptr[col + 1];
        if (b - a > kTrimLen) {
          int32_t lo = lower_bound_dev(row_ind, a, b, cs);
          int32_t hi = lower_bound_dev(row_ind, lo, b, ce);
          a = lo;
          b = hi;
        }
      }
      const int32_t len = b - a;
      const int32_t incl = wave_incl_scan(len);
      const int32_t excl = incl - len;
      const int32_t total = readlane(incl, kWave - 1);
      for (int32_t f0 = 0; f0 < total; f0 += kWave) {
        const int32_t f = f0 + lane;
        // Largest segment j with excl[j] <= f (excl is non-decreasing).
        int32_t j = 0;
#pragma unroll
        for (int step = 32; step > 0; step >>= 1) {
          int32_t t = j + step;
          int32_t e = __shfl(excl, t & (kWave - 1), kWave);
          if (t < kWave && e <= f) j = t;
        }
        const int32_t seg_a = __shfl(a, j, kWave);
        const int32_t seg_x = __shfl(excl, j, kWave);
        bool item = false;
        int32_t other = -1;
        float alpha = 0.0f;
        if (f < total) {
          other = row_ind[seg_a + (f - seg_x)];
          if (other >= cs && other < ce && other != row) {
            int32_t sz = row_ptr[other + 1] - row_ptr[other];
            alpha = 2.0f / static_cast<float>(row_size + sz);
            item = true;
          }
        }
        uint64_t mask = ballot(item);
        while (mask) {
          int i = __builtin_ctzll(mask);
          store.add(readlane(other, i), readlane_f(alpha, i));
          mask &= mask - 1;
        }
      }
    }
    store.select_top_k(k, out);
  }
}

template <int CELLS>
void launch_sketch(Context &ctx, int32_t n, int32_t k, int32_t chunk_size,
                   const int32_t *d_ptr, const int32_t *d_ind,
                   const int32_t *d_col_ptr, const int32_t *d_row_ind,
                   uint64_t *d_table) {
  int g = ctx.grid_for(ceil_div64(n, kSketchWaves), kSketchBlock, 4);
  chunk_sketch_kernel<CELLS><<<g, kSketchBlock, 0, ctx.stream>>>(
      n, k, chunk_size, d_ptr, d_ind, d_col_ptr, d_row_ind, d_table);
  SP_LAUNCH_CHECK();
}

// ---- greedy chain ----------------------------------------------------------

struct ChainCounters {
  int32_t restarts;
  int32_t links;
  double link_weight_sum;
};

constexpr int kGreedyBlock = 256;
constexpr int kGreedyWaves = kGreedyBlock / kWave;

// One wave per chunk.  `words_per_wave` u32 words of visited bitmap per wave
// live in LDS (use_lds) or in `gbitmap` at chunk * words_per_wave.
__global__ void __launch_bounds__(kGreedyBlock)
    greedy_kernel(int32_t n, int32_t k, int32_t chunk_size, int32_t num_chunks,
                  const uint64_t *__restrict__ table, int32_t *__restrict__ order,
                  ChainCounters *counters, uint32_t *gbitmap,
                  int32_t words_per_wave, int use_lds) {
  extern __shared__ uint32_t lds_bitmap[];
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int64_t chunk = static_cast<int64_t>(blockIdx.x) * kGreedyWaves + wave;
  if (chunk >= num_chunks) return;
  const int64_t start64 = chunk * chunk_size;
  const int32_t start = static_cast<int32_t>(start64);
  const int32_t end =
      static_cast<int32_t>(start64 + chunk_size > n ? n : start64 + chunk_size);
  if (start >= end) return;
  const int32_t size = end - start;
  const int32_t words = (size + 31) >> 5;
  uint32_t *bm = use_lds ? lds_bitmap + static_cast<size_t>(wave) * words_per_wave
                         : gbitmap + static_cast<size_t>(chunk) * words_per_wave;
  for (int32_t w = lane; w < words; w += kWave) bm[w] = 0u;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  const uint32_t tail_mask =
      (size & 31) ? ((1u << (size & 31)) - 1u) : 0xFFFFFFFFu;
  int32_t cur = start, pos = start, low_word = 0;
  int32_t restarts = 0, links = 0;
  float link_w = 0.0f;

  while (true) {
    if (lane == 0) {
      int32_t b = cur - start;
      bm[b >> 5] |= 1u << (b & 31);
      order[pos] = cur;
    }
    pos += 1;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    const uint64_t *row = table + static_cast<size_t>(cur) * k;
    float best_w = -1.0f;
    int32_t best_c = -1;
    for (int32_t j = lane; j < k; j += kWave) {
      uint64_t e = row[j];
      int32_t cand = wi_index(e);
      if (cand < 0) break; // valid entries form a prefix
      if (cand < start || cand >= end) continue;
      int32_t b = cand - start;
      if (bm[b >> 5] & (1u << (b & 31))) continue;
      float w = wi_weight(e);
      if (w > best_w || (w == best_w && cand < best_c)) {
        best_w = w;
        best_c = cand;
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      float ow = __shfl_xor(best_w, off, kWave);
      int32_t oc = __shfl_xor(best_c, off, kWave);
      if (ow > best_w || (ow == best_w && oc < best_c)) {
        best_w = ow;
        best_c = oc;
      }
    }
    best_c = __builtin_amdgcn_readfirstlane(best_c);
    if (best_c >= 0) {
      links += 1;
      link_w += readlane_f(best_w, 0);
      cur = best_c;
      continue;
    }
    // Restart at the lowest unvisited row; it never moves backwards.
    int32_t nxt = -1;
    while (low_word < words) {
      int32_t w = low_word + lane;
      uint32_t free_bits = 0u;
      if (w < words) {
        free_bits = ~bm[w] & (w == words - 1 ? tail_mask : 0xFFFFFFFFu);
      }
      uint64_t m = ballot(free_bits != 0u);
      if (m) {
        int first = __builtin_ctzll(m);
        uint32_t fb = static_cast<uint32_t>(readlane(static_cast<int32_t>(free_bits), first));
        low_word += first;
        nxt = low_word * 32 + __builtin_ctz(fb);
        break;
      }
      low_word += kWave;
    }
    if (nxt < 0) break;
    restarts += 1;
    cur = start + nxt;
  }
  if (counters != nullptr && lane == 0) {
    atomicAdd(&counters->restarts, restarts);
    atomicAdd(&counters->links, links);
    atomicAdd(&counters->link_weight_sum, static_cast<double>(link_w));
  }
}

// ---- table statistics -------------------------------------------------------

__global__ void __launch_bounds__(256)
    top_k_stats_kernel(int32_t n, int32_t k, const uint64_t *__restrict__ table,
                       TopKTotals *totals) {
  unsigned long long deg_sum = 0;
  double w_sum = 0.0;
  int32_t zeros = 0;
  for (int64_t row = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
       row < n; row += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const uint64_t *r = table + static_cast<size_t>(row) * k;
    int32_t degree = 0;
    float rw = 0.0f;
    for (int32_t j = 0; j < k; ++j) {
      uint64_t e = r[j];
      if (wi_index(e) == -1) break;
      degree += 1;
      rw += wi_weight(e);
    }
    deg_sum += degree;
    w_sum += rw;
    zeros += (degree == 0);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    deg_sum += __shfl_xor(deg_sum, off, kWave);
    w_sum += __shfl_xor(w_sum, off, kWave);
    zeros += __shfl_xor(zeros, off, kWave);
  }
  if (lane_id() == 0) {
    if (deg_sum > 0) {
      atomicAdd(&totals->total_degree, deg_sum);
      atomicAdd(&totals->total_weight, w_sum);
    }
    if (zeros > 0) atomicAdd(&totals->zero_degree_rows, zeros);
  }
}

__global__ void unpack_table_kernel(int64_t count, const uint64_t *__restrict__ t,
                                    int32_t *__restrict__ idx,
                                    float *__restrict__ w) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
       i < count; i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    uint64_t e = t[i];
    idx[i] = wi_index(e);
    w[i] = wi_weight(e);
  }
}

void zero_words(Context &ctx, void *p, size_t bytes) {
  fill_u32(ctx, p, static_cast<int64_t>(bytes / 4), 0u);
}

int32_t sketch_m(int32_t k, float oversampling) {
  int32_t m = static_cast<int32_t>(k * oversampling);
  return ((m + 31) / 32) * 32;
}

void validate_sketch_args(int32_t k, float oversampling, int32_t chunk_size) {
  // Reference: sporder/src/common/chunk_similarity_top_k.cu:143-147.
  SP_EXPECT(k > 0, "expect k > 0");
  SP_EXPECT(oversampling >= 1, "expect oversampling >= 1");
  SP_EXPECT(chunk_size >= 1, "expect chunk_size >= 1");
  int32_t m = static_cast<int32_t>(k * oversampling);
  SP_EXPECT(m <= 512, "expect k * oversampling <= 512");
}

// Workspace of the sketch stage: table + optional CSC.
size_t sketch_ws_bytes(int32_t n, int32_t nnz, int32_t k, bool is_symmetric) {
  size_t b = ws_bytes<uint64_t>(static_cast<size_t>(n) * k);
  if (!is_symmetric) {
    b += ws_bytes<int32_t>(static_cast<size_t>(n) + 1) +
         ws_bytes<int32_t>(static_cast<size_t>(nnz)) + csr2csc_ws_bytes(n, nnz);
  }
  return b;
}

struct ResolvedCsc {
  const int32_t *ptr;
  const int32_t *ind;
};

ResolvedCsc resolve_csc(Context &ctx, int32_t n, int32_t nnz, const int32_t *d_ptr,
                        const int32_t *d_ind, bool is_symmetric) {
  // Reference: sporder/src/common/csr2csc.h:49-59.
  if (is_symmetric) return {d_ptr, d_ind};
  int32_t *cp = ctx.take<int32_t>(static_cast<size_t>(n) + 1);
  int32_t *ri = ctx.take<int32_t>(static_cast<size_t>(nnz));
  csr2csc(ctx, n, nnz, d_ptr, d_ind, cp, ri);
  return {cp, ri};
}

} // namespace

void chunk_sketch_top_k(Context &ctx, int32_t n, int32_t k, int32_t chunk_size,
                        int32_t m_capacity, const int32_t *d_ptr,
                        const int32_t *d_ind, const int32_t *d_col_ptr,
                        const int32_t *d_row_ind, uint64_t *d_table) {
  SP_EXPECT(k <= 256, "k must be <= 256");
  switch (m_capacity / 32) {
#define SP_CASE(C)                                                             \
  case C:                                                                      \
    launch_sketch<C>(ctx, n, k, chunk_size, d_ptr, d_ind, d_col_ptr,           \
                     d_row_ind, d_table);                                      \
    break;
    SP_CASE(1) SP_CASE(2) SP_CASE(3) SP_CASE(4) SP_CASE(5) SP_CASE(6)
    SP_CASE(7) SP_CASE(8) SP_CASE(9) SP_CASE(10) SP_CASE(11) SP_CASE(12)
    SP_CASE(13) SP_CASE(14) SP_CASE(15) SP_CASE(16)
#undef SP_CASE
  default:
    SP_EXPECT(false, "sketch capacity must be a multiple of 32 in [32, 512]");
  }
}

void top_k_stats(Context &ctx, int32_t n, int32_t k, const uint64_t *d_table,
                 TopKTotals *d_totals) {
  int g = ctx.grid_for(ceil_div64(n, 256), 256, 4);
  top_k_stats_kernel<<<g, 256, 0, ctx.stream>>>(n, k, d_table, d_totals);
  SP_LAUNCH_CHECK();
}

} // namespace sporder_hip

using namespace sporder_hip;

extern "C" {

void sporder_chunk_similarity_greedy(sporder_context_t h, int32_t n,
                                     int32_t nnz, const int32_t *d_ptr,
                                     const int32_t *d_ind, bool is_symmetric,
                                     int32_t k, float oversampling,
                                     int32_t chunk_size, int32_t *d_new_order,
                                     sporder_csg_timing_t *timing,
                                     sporder_csg_stats_t *stats) {
  auto wall0 = std::chrono::steady_clock::now();
  SP_EXPECT(h != nullptr, "null context");
  SP_EXPECT(n >= 1 && nnz >= 0, "expect n >= 1 and nnz >= 0");
  Context &ctx = h->impl;
  // Defaults: reference sporder/src/sporder.cpp:147-161.
  if (k <= 0) k = std::min(256, std::max(16, 1 * (nnz / n)));
  if (oversampling <= 0.0f) oversampling = 4.0f;
  if (chunk_size <= 0) chunk_size = 1024;
  validate_sketch_args(k, oversampling, chunk_size);
  const int32_t m_cap = sketch_m(k, oversampling);
  if (stats) {
    stats->k_used = k;
    stats->m_used = m_cap;
    stats->chunk_size_used = chunk_size;
  }
  const int64_t num_chunks = ceil_div64(n, chunk_size);
  const int64_t words64 = ceil_div64(std::min<int64_t>(chunk_size, n), 32);
  SP_EXPECT(words64 < (int64_t(1) << 30), "chunk too large");
  const int32_t words = static_cast<int32_t>(words64);
  const size_t lds_need = static_cast<size_t>(words) * 4u;
  // Up to 4 chunks per workgroup share the LDS; very large chunks fall back
  // to a bitmap in the workspace.
  const bool use_lds = lds_need <= 64u * 1024u && lds_need <= ctx.lds_per_block;
  const int waves_per_block =
      use_lds ? static_cast<int>(std::max<size_t>(
                    1, std::min<size_t>(kGreedyWaves, (64u * 1024u) / std::max<size_t>(lds_need, 1))))
              : kGreedyWaves;

  size_t need = sketch_ws_bytes(n, nnz, k, is_symmetric) + ws_bytes<ChainCounters>(1) +
                ws_bytes<TopKTotals>(1);
  if (!use_lds) need += ws_bytes<uint32_t>(static_cast<size_t>(num_chunks) * words);
  ctx.reserve(need);
  uint64_t *table = ctx.take<uint64_t>(static_cast<size_t>(n) * k);
  ChainCounters *counters = ctx.take<ChainCounters>(1);
  TopKTotals *totals = ctx.take<TopKTotals>(1);
  uint32_t *gbitmap =
      use_lds ? nullptr : ctx.take<uint32_t>(static_cast<size_t>(num_chunks) * words);

  EventSpan t_csc, t_sim, t_greedy;
  t_csc.create(timing != nullptr);
  t_sim.create(timing != nullptr);
  t_greedy.create(timing != nullptr);

  if (stats) {
    // Zeroed by a kernel (not a memset node) so the call stays capturable.
    zero_words(ctx, counters, sizeof(ChainCounters));
    zero_words(ctx, totals, sizeof(TopKTotals));
  }

  t_csc.begin(ctx.stream);
  ResolvedCsc csc = resolve_csc(ctx, n, nnz, d_ptr, d_ind, is_symmetric);
  t_csc.end(ctx.stream);

  t_sim.begin(ctx.stream);
  chunk_sketch_top_k(ctx, n, k, chunk_size, m_cap, d_ptr, d_ind, csc.ptr, csc.ind,
                     table);
  t_sim.end(ctx.stream);
  if (stats) top_k_stats(ctx, n, k, table, totals);

  t_greedy.begin(ctx.stream);
  {
    int wpb = use_lds ? waves_per_block : kGreedyWaves;
    int64_t blocks = ceil_div64(num_chunks, wpb);
    size_t lds = use_lds ? static_cast<size_t>(wpb) * words * 4u : 0;
    greedy_kernel<<<dim3(static_cast<unsigned>(blocks)), wpb * kWave, lds,
                    ctx.stream>>>(n, k, chunk_size, static_cast<int32_t>(num_chunks),
                                  table, d_new_order, stats ? counters : nullptr,
                                  gbitmap, words, use_lds ? 1 : 0);
    SP_LAUNCH_CHECK();
  }
  t_greedy.end(ctx.stream);

  ChainCounters hc{};
  TopKTotals ht{};
  if (stats) {
    SP_HIP(hipMemcpyAsync(&hc, counters, sizeof(hc), hipMemcpyDeviceToHost,
                          ctx.stream));
    SP_HIP(hipMemcpyAsync(&ht, totals, sizeof(ht), hipMemcpyDeviceToHost,
                          ctx.stream));
  }
  ctx.sync();

  if (stats) {
    // Reference: sporder/src/csg/stats_collector.cu:43-63.
    stats->avg_degree = static_cast<double>(ht.total_degree) / n;
    stats->avg_edge_weight =
        ht.total_degree > 0 ? ht.total_weight / static_cast<double>(ht.total_degree)
                            : 0.0;
    stats->zero_degree_rows = ht.zero_degree_rows;
    stats->chain_restarts = hc.restarts;
    stats->avg_followed_weight =
        hc.links > 0 ? hc.link_weight_sum / hc.links : 0.0;
  }
  if (timing) {
    timing->csr2csc_ms = t_csc.ms();
    timing->similarity_ms = t_sim.ms();
    timing->chunk_greedy_ms = t_greedy.ms();
    timing->wall_ms = std::chrono::duration<double, std::milli>(
                          std::chrono::steady_clock::now() - wall0)
                          .count();
  }
  t_csc.destroy();
  t_sim.destroy();
  t_greedy.destroy();
}

void sporder_chunk_similarity_top_k(sporder_context_t h, int32_t n, int32_t nnz,
                                    const int32_t *d_ptr, const int32_t *d_ind,
                                    bool is_symmetric, int32_t k,
                                    float oversampling, int32_t chunk_size,
                                    int32_t *d_indices, float *d_weights) {
  SP_EXPECT(h != nullptr, "null context");
  SP_EXPECT(n >= 1 && nnz >= 0, "expect n >= 1 and nnz >= 0");
  validate_sketch_args(k, oversampling, chunk_size);
  Context &ctx = h->impl;
  ctx.reserve(sketch_ws_bytes(n, nnz, k, is_symmetric));
  uint64_t *table = ctx.take<uint64_t>(static_cast<size_t>(n) * k);
  ResolvedCsc csc = resolve_csc(ctx, n, nnz, d_ptr, d_ind, is_symmetric);
  chunk_sketch_top_k(ctx, n, k, chunk_size, sketch_m(k, oversampling), d_ptr, d_ind,
                     csc.ptr, csc.ind, table);
  int64_t count = static_cast<int64_t>(n) * k;
  int g = ctx.grid_for(ceil_div64(count, 256), 256, 4);
  unpack_table_kernel<<<g, 256, 0, ctx.stream>>>(count, table, d_indices, d_weights);
  SP_LAUNCH_CHECK();
  ctx.sync();
}

void sporder_similarity_graph(sporder_context_t h, int32_t n, int32_t nnz,
                              const int32_t *d_ptr, const int32_t *d_ind,
                              bool is_symmetric, int32_t k, float oversampling,
                              int32_t *d_indices, float *d_weights,
                              sporder_sim_timing_t *timing,
                              sporder_sim_stats_t *stats) {
  auto wall0 = std::chrono::steady_clock::now();
  SP_EXPECT(h != nullptr, "null context");
  SP_EXPECT(n >= 1 && nnz >= 0, "expect n >= 1 and nnz >= 0");
  Context &ctx = h->impl;
  // Defaults: reference sporder/src/sporder.cpp:75-85.
  if (k <= 0) k = std::min(32, std::max(16, 2 * (nnz / n)));
  if (oversampling <= 0.0f) oversampling = 2.0f;
  // One chunk spanning every row is the global sketch of
  // sporder/src/common/similarity_top_k.cu:10-51.
  validate_sketch_args(k, oversampling, n);
  const int32_t m_cap = sketch_m(k, oversampling);
  if (stats) {
    stats->k_used = k;
    stats->m_used = m_cap;
  }
  ctx.reserve(sketch_ws_bytes(n, nnz, k, is_symmetric) + ws_bytes<TopKTotals>(1));
  uint64_t *table = ctx.take<uint64_t>(static_cast<size_t>(n) * k);
  TopKTotals *totals = ctx.take<TopKTotals>(1);
  EventSpan t_csc, t_sim, t_unpack;
  t_csc.create(timing != nullptr);
  t_sim.create(timing != nullptr);
  t_unpack.create(timing != nullptr);

  t_csc.begin(ctx.stream);
  ResolvedCsc csc = resolve_csc(ctx, n, nnz, d_ptr, d_ind, is_symmetric);
  t_csc.end(ctx.stream);
  t_sim.begin(ctx.stream);
  chunk_sketch_top_k(ctx, n, k, n, m_cap, d_ptr, d_ind, csc.ptr, csc.ind, table);
  t_sim.end(ctx.stream);
  if (stats) {
    zero_words(ctx, totals, sizeof(TopKTotals));
    top_k_stats(ctx, n, k, table, totals);
  }
  int64_t count = static_cast<int64_t>(n) * k;
  int g = ctx.grid_for(ceil_div64(count, 256), 256, 4);
  t_unpack.begin(ctx.stream);
  unpack_table_kernel<<<g, 256, 0, ctx.stream>>>(count, table, d_indices, d_weights);
  SP_LAUNCH_CHECK();
  t_unpack.end(ctx.stream);
  TopKTotals ht{};
  if (stats) {
    SP_HIP(hipMemcpyAsync(&ht, totals, sizeof(ht), hipMemcpyDeviceToHost, ctx.stream));
  }
  ctx.sync();
  if (timing) {
    timing->csr2csc_ms = t_csc.ms();
    timing->similarity_ms = t_sim.ms();
    timing->unpack_ms = t_unpack.ms();
    timing->wall_ms = std::chrono::duration<double, std::milli>(
                          std::chrono::steady_clock::now() - wall0)
                          .count();
  }
  if (stats) {
    stats->avg_degree = static_cast<double>(ht.total_degree) / n;
    stats->avg_edge_weight =
        ht.total_degree > 0 ? ht.total_weight / static_cast<double>(ht.total_degree)
                            : 0.0;
    stats->zero_degree_rows = ht.zero_degree_rows;
  }
  t_csc.destroy();
  t_sim.destroy();
  t_unpack.destroy();
}

} // extern "C"
