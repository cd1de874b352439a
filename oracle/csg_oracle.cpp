// csg_oracle.cpp -- CPU restatement of the reference's Chunked Greedy
// (sporder-csg) path, its permutation apply and a CSR SpMM.
//
// TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
// library and the CPU baseline timed by bench.py.  Only tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg load it; the
// product path (chunkedgreedy_amd) never does.
//
// Every function restates the reference algorithm from its source, cited as
// file:line relative to the reference checkout.  Parity pins (what checks
// each function independently of this restatement) are listed per function.
//
// Build: g++ -O2 -std=c++17 -fopenmp -fno-fast-math -ffp-contract=off
//        -shared -fPIC (oracle/Makefile).  fp-contract=off keeps every fp32
// add a separate rounding, as in the reference's `+=` on float registers.

#include <algorithm>
#include <cmath>
#include <unordered_map>
#include <cstdint>
#include <cstring>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

// ---------------------------------------------------------------------------
// weighted_index packing.
// Follows sporder/src/common/weighted_index.h:15-27:
//   u64 = (bits(weight) << 32) | (uint32)(index + 1); index() = low32 - 1.
// A zeroed entry therefore reads as (index -1, weight +0.0).
// Pinned by: tests/test_oracle_golden.py (packing round trip, zero entry).
// ---------------------------------------------------------------------------
inline uint64_t pack_wi(int32_t index, float weight) {
  uint32_t wb;
  std::memcpy(&wb, &weight, 4);
  return (static_cast<uint64_t>(wb) << 32) |
         static_cast<uint32_t>(index + 1);
}
inline int32_t wi_index(uint64_t v) {
  return static_cast<int32_t>(static_cast<uint32_t>(v & 0xFFFFFFFFu)) - 1;
}
inline float wi_weight(uint64_t v) {
  uint32_t wb = static_cast<uint32_t>(v >> 32);
  float w;
  std::memcpy(&w, &wb, 4);
  return w;
}

// ---------------------------------------------------------------------------
// 32-lane space-saving sketch of capacity M = 32 * CELLS.
// Follows sporder/src/common/warp_spacesaving.cuh:
//   state          :12-29   (keys -1, weights 0 after clear)
//   add (per item) :31-44   (items of a 32-wide batch in ascending lane order)
//   single add     :109-150 (found -> +=; else lowest lane with an empty cell,
//                            its lowest empty cell; else evict the minimum
//                            weight, per-lane strict '<' then warp_arg_min with
//                            ties -> smaller (cell<<5 | lane); inherit weight)
//   select_top_k   :46-66   (per-lane selection sort :69-88, then k rounds of
//                            warp_arg_max over lane heads, ties -> smaller lane,
//                            exhausted lanes present 0.0f)
//   warp_arg_reduce: sporder/src/common/cuda_util.cuh:66-87
// The restatement keeps the literal [lane][cell] layout of the reference so
// that every tie rule reads off the source directly.
// Pinned by: the no-eviction closed form (tests/test_oracle_sketch.py, an
// independent count/first-occurrence computation), hand-worked eviction
// fixtures (tests/golden/sketch_cases.json) and the band-matrix known answer
// derived from sporder/tests/smoke.c:58-70 (tests/golden/band_kat.json).
// ---------------------------------------------------------------------------
struct SpaceSaving {
  int cells;
  std::vector<int32_t> keys;  // [32][cells]
  std::vector<float> weights; // [32][cells]
  // key -> lane*cells + c for the keys present: an index over `keys` that
  // makes find() O(1); it never changes which slot a key is found in.
  std::unordered_map<int32_t, int> where;

  explicit SpaceSaving(int m) : cells(m / 32), keys(m), weights(m) { clear(); }

  int32_t &key(int lane, int c) { return keys[lane * cells + c]; }
  float &wt(int lane, int c) { return weights[lane * cells + c]; }

  void clear() {
    std::fill(keys.begin(), keys.end(), -1);
    std::fill(weights.begin(), weights.end(), 0.0f);
    where.clear();
  }

  void single_add(int32_t k, float w) {
    // (i) existing key: weight += w (warp_spacesaving.cuh:111-119)
    auto it = where.find(k);
    if (it != where.end()) {
      weights[it->second] += w;
      return;
    }
    // (ii) lowest lane with an empty cell, that lane's first empty cell
    //      (:121-131; find(-1) is the first cell holding -1)
    if (where.size() < keys.size()) {
      for (int lane = 0; lane < 32; ++lane) {
        for (int c = 0; c < cells; ++c) {
          if (key(lane, c) == -1) {
            key(lane, c) = k;
            wt(lane, c) = w;
            where[k] = lane * cells + c;
            return;
          }
        }
      }
    }
    // (iii) evict the minimum (:133-149)
    int best_key = 0;
    float best_w = 0.0f;
    for (int lane = 0; lane < 32; ++lane) {
      int lane_key = (0 << 5) | lane;
      float lane_min = wt(lane, 0);
      for (int c = 1; c < cells; ++c) {
        if (wt(lane, c) < lane_min) {
          lane_min = wt(lane, c);
          lane_key = (c << 5) | lane;
        }
      }
      // warp_arg_min: smaller value wins; equal values -> smaller key
      if (lane == 0 || lane_min < best_w ||
          (lane_min == best_w && lane_key < best_key)) {
        best_w = lane_min;
        best_key = lane_key;
      }
    }
    int lane = best_key & 31, c = best_key >> 5;
    where.erase(key(lane, c));
    key(lane, c) = k;
    wt(lane, c) += w; // the new key inherits the evicted weight
    where[k] = lane * cells + c;
  }

  void local_sort_descending(int lane) {
    for (int i = 0; i < cells - 1; ++i) {
      int best = i;
      if (key(lane, best) == -1) {
        break;
      }
      for (int j = i + 1; j < cells; ++j) {
        if (key(lane, j) == -1) {
          break;
        }
        if (wt(lane, j) > wt(lane, best)) {
          best = j;
        }
      }
      if (best != i) {
        std::swap(key(lane, i), key(lane, best));
        std::swap(wt(lane, i), wt(lane, best));
      }
    }
  }

  // Writes up to k entries to out[0..k); entries not written keep their
  // previous contents (the reference pre-zeroes the table).
  void select_top_k(int k, uint64_t *out) {
    for (int lane = 0; lane < 32; ++lane) {
      local_sort_descending(lane);
    }
    int pos[32] = {0};
    for (int i = 0; i < k; ++i) {
      bool all_done = true;
      for (int lane = 0; lane < 32; ++lane) {
        if (!(pos[lane] >= cells || key(lane, pos[lane]) == -1)) {
          all_done = false;
        }
      }
      if (all_done) {
        break;
      }
      int best_lane = 0;
      float best_w = 0.0f;
      for (int lane = 0; lane < 32; ++lane) {
        float v = pos[lane] < cells ? wt(lane, pos[lane]) : 0.0f;
        // warp_arg_max: larger value wins; equal values -> smaller lane
        if (lane == 0 || v > best_w) {
          best_w = v;
          best_lane = lane;
        }
      }
      out[i] = pack_wi(key(best_lane, pos[best_lane]),
                       wt(best_lane, pos[best_lane]));
      pos[best_lane] += 1;
    }
  }
};

int32_t sketch_capacity(int32_t k, float oversampling) {
  // m = (int)(k * oversampling) rounded up to a multiple of 32
  // (chunk_similarity_top_k.cu:146 and dispatch :111-135, which selects the
  // smallest instantiated M >= m; sporder.cpp:159 reports the same value).
  int32_t m = static_cast<int32_t>(k * oversampling);
  return ((m + 31) / 32) * 32;
}

} // namespace

extern "C" {

// ---------------------------------------------------------------------------
// Defaults bridge.  Follows sporder/src/sporder.cpp:147-161:
//   k <= 0 -> min(256, max(16, nnz / n)); ovs <= 0 -> 4.0; chunk <= 0 -> 1024;
//   m_used = ((int)(k * ovs) + 31) / 32 * 32.
// Pinned by: closed forms in tests/test_oracle_golden.py (config table values).
// ---------------------------------------------------------------------------
void oracle_csg_defaults(int32_t n, int32_t nnz, int32_t k, float ovs,
                         int32_t chunk, int32_t *k_out, float *ovs_out,
                         int32_t *chunk_out, int32_t *m_out) {
  if (k <= 0) {
    k = std::min(256, std::max(16, 1 * (nnz / n)));
  }
  if (ovs <= 0.0f) {
    ovs = 4.0f;
  }
  if (chunk <= 0) {
    chunk = 1024;
  }
  *k_out = k;
  *ovs_out = ovs;
  *chunk_out = chunk;
  *m_out = ((static_cast<int32_t>(k * ovs) + 31) / 32) * 32;
}

// ---------------------------------------------------------------------------
// Stable CSR -> CSC transpose: rows ascend within each column.
// Follows sporder/src/common/csr2csc.cu:38-115 (stable radix sort of
// (col, row) pairs + histogram + exclusive scan).
// Pinned by: scipy tocsc() with sorted indices (tests/test_oracle_csr.py).
// ---------------------------------------------------------------------------
void oracle_csr2csc(int32_t n, int32_t nnz, const int32_t *ptr,
                    const int32_t *ind, int32_t *col_ptr, int32_t *row_ind) {
  std::vector<int64_t> cnt(static_cast<size_t>(n) + 1, 0);
  for (int64_t p = 0; p < nnz; ++p) {
    cnt[ind[p] + 1] += 1;
  }
  for (int32_t c = 0; c < n; ++c) {
    cnt[c + 1] += cnt[c];
  }
  for (int32_t c = 0; c <= n; ++c) {
    col_ptr[c] = static_cast<int32_t>(cnt[c]);
  }
  std::vector<int64_t> fill(cnt.begin(), cnt.end() - 1);
  for (int32_t r = 0; r < n; ++r) {
    for (int32_t p = ptr[r]; p < ptr[r + 1]; ++p) {
      row_ind[fill[ind[p]]++] = r;
    }
  }
}

// ---------------------------------------------------------------------------
// Chunk-restricted sketch + top-k (the csg similarity stage).
// Follows sporder/src/common/chunk_similarity_top_k.cu:30-88,137-154:
//   rows with |r| = 0 are skipped; chunk = [r/C*C, min(r/C*C + C, n));
//   stream = for each column c of r in CSR order, for each row s of column c
//   in CSC order with chunk_start <= s < chunk_end and s != r, item
//   (s, 2.0f / (float)(|r| + |s|)).  The lower_bound start (:59-63) and the
//   __all_sync break (:79-82) only skip items the filter rejects.
// `table` (n*k u64) is zeroed first (:150).  chunk_size = n reproduces the
// global sketch of sporder/src/common/similarity_top_k.cu:10-51.
// Pinned by: brute-force stream enumeration and the no-eviction closed form
// (tests/test_oracle_sketch.py), the band known answer, eviction fixtures.
// ---------------------------------------------------------------------------
int32_t oracle_chunk_similarity_top_k(int32_t n, int32_t k, int32_t chunk_size,
                                      float oversampling, const int32_t *ptr,
                                      const int32_t *ind,
                                      const int32_t *col_ptr,
                                      const int32_t *row_ind,
                                      uint64_t *table) {
  if (k <= 0 || oversampling < 1.0f || chunk_size < 1) {
    return -1;
  }
  int32_t m = static_cast<int32_t>(k * oversampling);
  if (m > 512) {
    return -2;
  }
  int32_t M = sketch_capacity(k, oversampling);
  std::memset(table, 0, sizeof(uint64_t) * static_cast<size_t>(n) * k);

#pragma omp parallel
  {
    SpaceSaving store(M);
#pragma omp for schedule(dynamic, 256)
    for (int32_t row = 0; row < n; ++row) {
      int32_t rs = ptr[row], re = ptr[row + 1];
      int32_t row_size = re - rs;
      if (row_size == 0) {
        continue;
      }
      int32_t cs = (row / chunk_size) * chunk_size;
      int32_t ce = cs + chunk_size;
      if (ce > n || ce < cs) {
        ce = n;
      }
      store.clear();
      for (int32_t p = rs; p < re; ++p) {
        int32_t col = ind[p];
        for (int32_t q = col_ptr[col]; q < col_ptr[col + 1]; ++q) {
          int32_t other = row_ind[q];
          if (other >= cs && other < ce && other != row) {
            int32_t sz = ptr[other + 1] - ptr[other];
            float alpha = 2.0f / static_cast<float>(row_size + sz);
            store.single_add(other, alpha);
          }
        }
      }
      store.select_top_k(k, table + static_cast<size_t>(row) * k);
    }
  }
  return M;
}

// ---------------------------------------------------------------------------
// Space-saving over an explicit item stream (one row), for hand-built cases.
// Same rules as above; out[0..k) is zeroed first.
// ---------------------------------------------------------------------------
void oracle_sketch_stream(int32_t m_capacity, int32_t k, int32_t count,
                          const int32_t *keys, const float *weights,
                          uint64_t *out) {
  SpaceSaving store(m_capacity);
  for (int32_t i = 0; i < count; ++i) {
    if (keys[i] != -1) {
      store.single_add(keys[i], weights[i]);
    }
  }
  std::memset(out, 0, sizeof(uint64_t) * k);
  store.select_top_k(k, out);
}

// ---------------------------------------------------------------------------
// Greedy chain per chunk.
// Follows sporder/src/csg/chunk_similarity_greedy.cu:14-98 and the bitmap
// sporder/src/common/warp_visited_bitmap.cuh:99-110:
//   cur = start; loop { mark cur; order[pos++] = cur;
//     best over row cur's entries (32 lanes, lane L scans j = L, L+32, ...
//     and stops at its first index < 0) with start <= s < end, s unvisited:
//     max weight, ties -> smaller index (warp_arg_max);
//     found -> cur = best (links += 1, per-chunk float link_weight_sum += w);
//     else cur = lowest unvisited in the chunk (restarts += 1) or stop }.
// Counters: restarts and links summed; link_weight_sum summed as double of
// per-chunk float sums (:88-95).
// Pinned by: brute-force nearest-neighbour chain on hand-written tables and
// invariants (tests/test_oracle_greedy.py).
// ---------------------------------------------------------------------------
void oracle_greedy(int32_t n, int32_t k, int32_t chunk_size,
                   const uint64_t *table, int32_t *order, int64_t *restarts_out,
                   int64_t *links_out, double *link_weight_out) {
  int32_t num_chunks = static_cast<int32_t>(
      (static_cast<int64_t>(n) + chunk_size - 1) / chunk_size);
  int64_t restarts_total = 0, links_total = 0;
  double lw_total = 0.0;
#pragma omp parallel for schedule(dynamic, 4) reduction(+ : restarts_total, links_total, lw_total)
  for (int32_t chunk = 0; chunk < num_chunks; ++chunk) {
    int64_t start64 = static_cast<int64_t>(chunk) * chunk_size;
    int32_t start = static_cast<int32_t>(start64);
    int32_t end = static_cast<int32_t>(std::min<int64_t>(start64 + chunk_size, n));
    if (start >= end) {
      continue;
    }
    std::vector<char> visited(end - start, 0);
    int32_t cur = start, pos = start, lowest = 0;
    int64_t restarts = 0, links = 0;
    float lw = 0.0f;
    while (true) {
      visited[cur - start] = 1;
      order[pos++] = cur;
      const uint64_t *row = table + static_cast<size_t>(cur) * k;
      float best_w = -1.0f;
      int32_t best_c = -1;
      for (int lane = 0; lane < 32; ++lane) {
        float lane_w = -1.0f;
        int32_t lane_c = -1;
        for (int32_t j = lane; j < k; j += 32) {
          int32_t cand = wi_index(row[j]);
          if (cand < 0) {
            break;
          }
          if (cand < start || cand >= end) {
            continue;
          }
          if (visited[cand - start]) {
            continue;
          }
          float w = wi_weight(row[j]);
          if (w > lane_w || (w == lane_w && cand < lane_c)) {
            lane_w = w;
            lane_c = cand;
          }
        }
        // warp_arg_max over (key = lane_c, value = lane_w)
        if (lane == 0 || lane_w > best_w ||
            (lane_w == best_w && lane_c < best_c)) {
          best_w = lane_w;
          best_c = lane_c;
        }
      }
      if (best_c >= 0) {
        links += 1;
        lw += best_w;
        cur = best_c;
        continue;
      }
      while (lowest < end - start && visited[lowest]) {
        ++lowest;
      }
      if (lowest >= end - start) {
        break;
      }
      restarts += 1;
      cur = start + lowest;
    }
    restarts_total += restarts;
    links_total += links;
    lw_total += static_cast<double>(lw);
  }
  *restarts_out = restarts_total;
  *links_out = links_total;
  *link_weight_out = lw_total;
}

// ---------------------------------------------------------------------------
// Top-k graph statistics.
// Follows sporder/src/common/similarity_top_k.cu:120-159 (degree = valid
// prefix length; per-row float weight sum in entry order; totals in u64 and
// double) and sporder/src/csg/stats_collector.cu:43-63 (averages).
// ---------------------------------------------------------------------------
void oracle_top_k_stats(int32_t n, int32_t k, const uint64_t *table,
                        uint64_t *total_degree, double *total_weight,
                        int32_t *zero_degree_rows) {
  uint64_t deg_total = 0;
  double w_total = 0.0;
  int64_t zeros = 0;
#pragma omp parallel for schedule(static) reduction(+ : deg_total, w_total, zeros)
  for (int32_t row = 0; row < n; ++row) {
    const uint64_t *r = table + static_cast<size_t>(row) * k;
    int32_t degree = 0;
    float rw = 0.0f;
    for (int32_t j = 0; j < k; ++j) {
      if (wi_index(r[j]) == -1) {
        break;
      }
      degree += 1;
      rw += wi_weight(r[j]);
    }
    deg_total += degree;
    w_total += rw;
    zeros += (degree == 0);
  }
  *total_degree = deg_total;
  *total_weight = w_total;
  *zero_degree_rows = static_cast<int32_t>(zeros);
}

// Stats block mirroring sporder_csg_stats_t (sporder/include/sporder.h:213-222).
struct oracle_csg_stats {
  int32_t k_used;
  int32_t m_used;
  double avg_degree;
  double avg_edge_weight;
  int32_t zero_degree_rows;
  int32_t chunk_size_used;
  int32_t chain_restarts;
  double avg_followed_weight;
};

// ---------------------------------------------------------------------------
// Whole csg pipeline.  Follows sporder/src/sporder.cpp:140-166 (defaults) and
// sporder/src/csg/chunk_similarity_greedy.cu:100-138 (csc -> sketch ->
// greedy).  is_symmetric aliases the CSR as CSC (csr2csc.h:49-59).
// Returns 0 on success, < 0 on an argument the reference rejects with expect.
// `table_out` may be NULL; otherwise it receives the n*k sketch table.
// ---------------------------------------------------------------------------
int32_t oracle_chunk_similarity_greedy(int32_t n, int32_t nnz,
                                       const int32_t *ptr, const int32_t *ind,
                                       int32_t is_symmetric, int32_t k,
                                       float oversampling, int32_t chunk_size,
                                       int32_t *new_order, uint64_t *table_out,
                                       oracle_csg_stats *stats) {
  int32_t m_used;
  oracle_csg_defaults(n, nnz, k, oversampling, chunk_size, &k, &oversampling,
                      &chunk_size, &m_used);
  std::vector<int32_t> cptr_buf, rind_buf;
  const int32_t *cptr = ptr, *rind = ind;
  if (!is_symmetric) {
    cptr_buf.resize(static_cast<size_t>(n) + 1);
    rind_buf.resize(std::max<int64_t>(nnz, 1));
    oracle_csr2csc(n, nnz, ptr, ind, cptr_buf.data(), rind_buf.data());
    cptr = cptr_buf.data();
    rind = rind_buf.data();
  }
  std::vector<uint64_t> own_table;
  uint64_t *table = table_out;
  if (!table) {
    own_table.resize(static_cast<size_t>(n) * k);
    table = own_table.data();
  }
  int32_t rc = oracle_chunk_similarity_top_k(n, k, chunk_size, oversampling,
                                             ptr, ind, cptr, rind, table);
  if (rc < 0) {
    return rc;
  }
  int64_t restarts = 0, links = 0;
  double lw = 0.0;
  oracle_greedy(n, k, chunk_size, table, new_order, &restarts, &links, &lw);
  if (stats) {
    uint64_t deg = 0;
    double wsum = 0.0;
    int32_t zeros = 0;
    oracle_top_k_stats(n, k, table, &deg, &wsum, &zeros);
    stats->k_used = k;
    stats->m_used = m_used;
    stats->chunk_size_used = chunk_size;
    stats->avg_degree = n > 0 ? static_cast<double>(deg) / n : 0.0;
    stats->avg_edge_weight = deg > 0 ? wsum / static_cast<double>(deg) : 0.0;
    stats->zero_degree_rows = zeros;
    stats->chain_restarts = static_cast<int32_t>(restarts);
    stats->avg_followed_weight = links > 0 ? lw / static_cast<double>(links) : 0.0;
  }
  return 0;
}

// ---------------------------------------------------------------------------
// Permutation apply.  Follows sporder/src/reorder.cu:72-149:
//   ROWS (mode 0): new row p = old row new_order[p], verbatim;
//   SYMMETRIC (mode 1): columns remapped by old2new, each row re-sorted by
//   column with values following.  ptr_new = inclusive scan of gathered
//   lengths.  val_new may be non-NULL with val_old NULL: ROWS then writes
//   zeros (gather_rows :37-45), SYMMETRIC leaves val_new untouched (:264-265).
// Pinned by: scipy A[perm,:] and A[perm,:][:,perm] with sorted indices
// (tests/test_oracle_csr.py).
// ---------------------------------------------------------------------------
void oracle_reorder(int32_t n, int32_t nnz, const int32_t *ptr_old,
                    const int32_t *ind_old, const float *val_old,
                    const int32_t *new_order, int32_t mode, int32_t *ptr_new,
                    int32_t *ind_new, float *val_new) {
  (void)nnz;
  ptr_new[0] = 0;
  for (int32_t p = 0; p < n; ++p) {
    int32_t o = new_order[p];
    ptr_new[p + 1] = ptr_new[p] + (ptr_old[o + 1] - ptr_old[o]);
  }
  bool symmetric = mode == 1;
  bool with_vals = val_old != nullptr && val_new != nullptr;
  std::vector<int32_t> old2new;
  if (symmetric) {
    old2new.resize(n);
    for (int32_t p = 0; p < n; ++p) {
      old2new[new_order[p]] = p;
    }
  }
#pragma omp parallel for schedule(dynamic, 1024)
  for (int32_t p = 0; p < n; ++p) {
    int32_t o = new_order[p];
    int32_t src = ptr_old[o], len = ptr_old[o + 1] - src, dst = ptr_new[p];
    if (!symmetric) {
      for (int32_t j = 0; j < len; ++j) {
        ind_new[dst + j] = ind_old[src + j];
        if (val_new) {
          val_new[dst + j] = val_old ? val_old[src + j] : 0.0f;
        }
      }
      continue;
    }
    std::vector<std::pair<int32_t, float>> row(len);
    for (int32_t j = 0; j < len; ++j) {
      row[j].first = old2new[ind_old[src + j]];
      row[j].second = with_vals ? val_old[src + j] : 0.0f;
    }
    std::stable_sort(row.begin(), row.end(),
                     [](const std::pair<int32_t, float> &a,
                        const std::pair<int32_t, float> &b) {
                       return a.first < b.first;
                     });
    for (int32_t j = 0; j < len; ++j) {
      ind_new[dst + j] = row[j].first;
      if (with_vals) {
        val_new[dst + j] = row[j].second;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// CSR SpMM, fp32, row-major B (n x N) and C (n x N), in the order the HIP
// row-split kernel states (include/sporder.h, SPORDER_SPMM_LONG_ROW and
// SPORDER_SPMM_SEGMENT):
//   - a row with at most long_row nonzeros: C[i][j] = fold over p in CSR order
//     of acc = fmaf(val[p], B[ind[p]][j], acc) from acc = 0.0f;
//   - a longer row: segments of seg_len nonzeros from the row start, each such
//     a fold from 0.0f, then C[i][j] = ((P0 + P1) + P2) + ... left to right.
// The reference's SpMM is cuSPARSE (closed source,
// sporder/src/bench_cusparse_spmm.cu:51-100); its accumulation order is not
// published, so parity with it is stated as fp64 A@B within 1e-5 relative.
// Pinned by: fp64 scipy A@B within tolerance, and each output against exact
// rational arithmetic rounded once per operation in the stated order, with a
// crafted row whose value depends on the segment boundary
// (tests/test_oracle_csr.py).
// ---------------------------------------------------------------------------
// part[j] = fmaf(a, b[j], part[j]) for j < N: one fused multiply-add per
// element, so lane-wise vector FMAs give the same bits as the scalar loop.
// Built for FMA-capable hosts and for a generic x86-64 one, chosen at load time.
__attribute__((target_clones("fma", "default"))) static void
fma_row(float a, const float *__restrict b, float *__restrict part, int32_t N) {
#pragma omp simd
  for (int32_t j = 0; j < N; ++j) {
    part[j] = std::fmaf(a, b[j], part[j]);
  }
}

void oracle_spmm_csr(int32_t n, const int32_t *ptr, const int32_t *ind,
                     const float *val, int32_t N, const float *B, float *C,
                     int32_t long_row, int32_t seg_len) {
#pragma omp parallel for schedule(dynamic, 256)
  for (int32_t i = 0; i < n; ++i) {
    float *crow = C + static_cast<size_t>(i) * N;
    const int32_t s = ptr[i], e = ptr[i + 1];
    const int32_t seg = (e - s > long_row) ? seg_len : (e - s > 0 ? e - s : 1);
    std::vector<float> part(static_cast<size_t>(N));
    for (int32_t q0 = s; q0 < e || q0 == s; q0 += seg) {
      const int32_t q1 = std::min(q0 + seg, e);
      for (int32_t j = 0; j < N; ++j) {
        part[j] = 0.0f;
      }
      for (int32_t p = q0; p < q1; ++p) {
        fma_row(val[p], B + static_cast<size_t>(ind[p]) * N, part.data(), N);
      }
      for (int32_t j = 0; j < N; ++j) {
        crow[j] = (q0 == s) ? part[j] : crow[j] + part[j];
      }
    }
  }
}

int32_t oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void oracle_set_num_threads(int32_t t) {
#ifdef _OPENMP
  if (t > 0) {
    omp_set_num_threads(t);
  }
#else
  (void)t;
#endif
}

} // extern "C"
