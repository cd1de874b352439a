// csg_local.hip -- chunk-local sketch + top-k: one workgroup per chunk, the
// chunk's transpose built in LDS.
//
// The reference computes the similarity of row r from the global CSC: for
// each column c of r (CSR order), the rows of c in ascending order, kept only
// when they fall inside r's chunk (sporder/src/common/chunk_similarity_top_k.cu
// :53-83).  Restricted to one chunk, those rows are exactly the chunk's own
// rows holding c, so the global transpose (a device-wide sort of every
// nonzero) and the random CSC walks are replaced by a transpose of the
// chunk's row block alone, in LDS:
//
//   1. every nonzero (c, local row) becomes the key (c << lb) | local_row and is
//      counting-sorted into buckets by a multiplicative hash of c (keys of one
//      column share a bucket; about 8 keys per bucket, up to the tier's
//      bucket capacity);
//   2. each bucket is sorted by key: one thread per bucket for small buckets
//      (a register bitonic network up to 16 keys, insertion sort up to 48),
//      one wave per bucket (bitonic network in LDS) for large ones.  A
//      column's keys are now one run, rows ascending;
//   3. a row whose columns all occur once in the chunk has no candidates and
//      gets the all-zero table row;
//   3b. the rows are counting-sorted by floor(log2(row size)), largest
//      first, rows without candidates last;
//   4. the workgroup writes the zero rows; waves claim the other rows in
//      order, and each binary-searches each column's run inside its bucket
//      and feeds the run's rows, ascending, to the wave64 sketch.
//
// The stream, and therefore the table, is identical to the reference's.
// Two LDS tiers: up to 16384 nonzeros, 1024 rows and 2048 buckets per chunk
// (~78 KiB, two workgroups per CU) and up to 32768 nonzeros, 4096 rows and
// 1024 buckets (~157 KiB).
// Larger chunks go to an overflow list for the global-CSC kernel.  Requires
// ceil(log2 n) + ceil(log2 C) <= 32 (checked by the host).
#include "common.hpp"
#include "sketch.hpp"
#include "wave_sort.hpp"

#include <algorithm>

namespace sporder_hip {

namespace {

constexpr int kLocalThreads = 1024;
constexpr int kLocalWaves = kLocalThreads / kWave;
// Buckets up to this size are sorted by one thread.
constexpr int kSmallBucket = 48;
// Column loads in flight per thread in the bucket count.
constexpr int kCountLoads = 8;
// Row classes of step 3b: clz(row size) in [0, 31] for rows with candidates,
// kClasses for the others.
constexpr int kClasses = 32;
// Step 3's mark: larger than any bucket id (< 2048) or row index (< 4096).
constexpr uint16_t kMultiMark = 0xFFFF;
constexpr int kRowsPerThread = kLocalRowCap / kLocalThreads;
// Tier 2 scatters rows of more nonzeros than this with a whole wave (step 2a).
constexpr int kScatterRowCap = 32;

__device__ __forceinline__ uint32_t bucket_of(uint32_t col, int nb_log2) {
  // Fibonacci hashing (Knuth, TAOCP vol. 3, 6.4): high bits of col * 2^32/phi.
  return (col * 0x9E3779B9u) >> (32 - nb_log2);
}

// First index in [lo, hi) with keys[i] >= bound.
__device__ __forceinline__ int32_t lds_lower_bound(const uint32_t *keys, int32_t lo,
                                                   int32_t hi, uint32_t bound) {
  while (lo < hi) {
    int32_t mid = (lo + hi) >> 1;
    if (keys[mid] < bound) {
      lo = mid + 1;
    } else {
      hi = mid;
    }
  }
  return lo;
}

// First index in [lo, hi) with keys[i] > bound.
__device__ __forceinline__ int32_t lds_upper_bound(const uint32_t *keys, int32_t lo,
                                                   int32_t hi, uint32_t bound) {
  while (lo < hi) {
    int32_t mid = (lo + hi) >> 1;
    if (keys[mid] <= bound) {
      lo = mid + 1;
    } else {
      hi = mid;
    }
  }
  return lo;
}

// Sorts keys[lo, lo + sz) (sz <= S) in one thread's registers with a bitonic
// network over S slots, padding with the largest key (equal keys are
// interchangeable, so a real key equal to the padding is still placed right).
template <int S>
__device__ __forceinline__ void register_sort_keys(uint32_t *keys, int32_t lo, int32_t sz) {
  uint32_t v[S];
#pragma unroll
  for (int i = 0; i < S; ++i) v[i] = i < sz ? keys[lo + i] : 0xFFFFFFFFu;
#pragma unroll
  for (int k = 2; k <= S; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
#pragma unroll
      for (int i = 0; i < S; ++i) {
        const int l = i ^ j;
        if (l > i) {
          const uint32_t a = v[i], c = v[l];
          const bool asc = (i & k) == 0;
          v[i] = asc ? min(a, c) : max(a, c);
          v[l] = asc ? max(a, c) : min(a, c);
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < S; ++i) {
    if (i < sz) keys[lo + i] = v[i];
  }
}

// Tier 1 (about 78 KiB of LDS) is sized for two workgroups per CU, which
// needs 8 waves per SIMD and so at most 64 VGPRs; the bound asks the
// compiler for that.  Capacities of 256 slots and more (CELLS >= 8) would
// spill to scratch under it and keep one workgroup per CU instead.
template <int CELLS, int KEYCAP>
constexpr int local_min_waves() {
  return (KEYCAP <= 16384 && CELLS <= 7) ? 8 : 1;
}

template <int CELLS, int KEYCAP, int ROWCAP, int NB_LOG2, bool CLAIM>
__global__ void __launch_bounds__(kLocalThreads, (local_min_waves<CELLS, KEYCAP>()))
    chunk_local_sketch_kernel(int32_t n, int32_t k, int32_t chunk_size, int32_t lb,
                              const int32_t *__restrict__ row_ptr,
                              const int32_t *__restrict__ col_ind,
                              uint64_t *__restrict__ table,
                              const int32_t *__restrict__ chunk_list,
                              const int32_t *__restrict__ chunk_list_count,
                              int32_t *__restrict__ overflow,
                              int32_t *__restrict__ overflow_count,
                              int32_t *__restrict__ row_valid,
                              unsigned long long *__restrict__ mirror,
                              uint32_t *__restrict__ claim) {
  constexpr int NB = 1 << NB_LOG2;
  static_assert(KEYCAP / (kSmallBucket + 1) <= ROWCAP, "large-bucket list must fit s_order");
  static_assert(NB <= kMultiMark && ROWCAP <= kMultiMark, "kMultiMark must be unused");
  // Tier 2 (the key capacity past 16384) scatters wide rows with a wave;
  // tier 1 runs at its register limit and keeps a thread per row.
  constexpr bool kWideRows = KEYCAP > 16384;
  __shared__ uint32_t s_keys[KEYCAP];
  __shared__ int32_t s_bend[NB];      // after the scatter: end of bucket b
  __shared__ int32_t s_size[ROWCAP];
  // Step 2b: the buckets too large for one thread; step 3: per-row "has a
  // candidate" marks (kMultiMark, a value no bucket id or row index takes);
  // from step 3b on: the chunk's rows in processing order.
  __shared__ uint16_t s_order[ROWCAP];
  __shared__ int32_t s_big_count;
  __shared__ int32_t s_slice_total[kLocalWaves]; // step 1's scan
  __shared__ int32_t s_class[kClasses + 1]; // counts, then cursors, per class
  __shared__ int32_t s_next_row;            // next entry of s_order to claim
  __shared__ unsigned long long s_mirror;   // this workgroup's mirror-check terms
  __shared__ uint32_t s_claimed[2];         // claimed list entries, by iteration parity

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;
  const uint32_t rmask = (lb == 0) ? 0u : ((1u << lb) - 1u);
  const int64_t num_chunks = ceil_div64(n, chunk_size);
  const int64_t work = chunk_list ? *chunk_list_count : num_chunks;

  for (int32_t r = threadIdx.x; r < ROWCAP; r += kLocalThreads) s_order[r] = 0;
  if (threadIdx.x == 0) s_mirror = 0;
  __syncthreads();
  // With CLAIM, workgroups claim list entries one at a time from `claim` (a
  // zeroed counter), so that workgroups placed late (beside another tier's,
  // until those leave) take fewer; without it they stride over the work.
  // The claimed entry sits in one of two words by iteration parity, so it is
  // not overwritten before every wave has read it (an iteration can end
  // without a barrier).
  auto next_entry = [&](int64_t it, int64_t t) -> int64_t {
    if constexpr (CLAIM) {
      if (tid == 0) s_claimed[it & 1] = atomicAdd(claim, 1u);
      __syncthreads();
      return s_claimed[it & 1];
    } else {
      return it == 0 ? static_cast<int64_t>(blockIdx.x) : t + gridDim.x;
    }
  };
  for (int64_t it = 0, t = next_entry(0, 0); t < work; ++it, t = next_entry(it, t)) {
    const int32_t chunk = chunk_list ? chunk_list[t] : static_cast<int32_t>(t);
    const int32_t cs = chunk * chunk_size;
    const int32_t ce = (n - cs > chunk_size) ? cs + chunk_size : n;
    const int32_t rows = ce - cs;
    const int32_t e0 = row_ptr[cs];
    const int32_t E = row_ptr[ce] - e0;
    if (E > KEYCAP || rows > ROWCAP) {
      // Another tier's chunk: listed here, or already listed by the
      // classification when `overflow` is null.
      if (tid == 0 && overflow != nullptr) overflow[atomicAdd(overflow_count, 1)] = chunk;
      continue; // uniform across the workgroup
    }
    // Buckets for about 8 keys each (at most NB, at least 64).
    int nbl = 6;
    while (nbl < NB_LOG2 && (E >> (nbl + 3)) > 0) ++nbl;
    const int32_t nb = 1 << nbl;

    // 1. Bucket counts (coalesced column reads) and row sizes.
    for (int32_t b = tid; b < nb; b += kLocalThreads) s_bend[b] = 0;
    if (tid <= kClasses) s_class[tid] = 0;
    if (tid == 0) {
      s_next_row = 0;
      s_big_count = 0;
    }
    for (int32_t r = tid; r < rows; r += kLocalThreads) {
      s_size[r] = row_ptr[cs + r + 1] - row_ptr[cs + r];
      // Valid counts start at zero, one coalesced store per row; the wave
      // that sketches a row overwrites its count after the barriers below.
      if (row_valid != nullptr) row_valid[cs + r] = 0;
    }
    __syncthreads();
    // kCountLoads coalesced column loads in flight per thread before their
    // atomics (one load at a time waited out the memory latency per key).
    for (int32_t i0 = tid; i0 < E; i0 += kCountLoads * kLocalThreads) {
      uint32_t c[kCountLoads];
#pragma unroll
      for (int u = 0; u < kCountLoads; ++u) {
        const int32_t i = i0 + u * kLocalThreads;
        c[u] = i < E ? static_cast<uint32_t>(col_ind[e0 + i]) : 0u;
      }
#pragma unroll
      for (int u = 0; u < kCountLoads; ++u) {
        if (i0 + u * kLocalThreads < E) atomicAdd(&s_bend[bucket_of(c[u], nbl)], 1);
      }
    }
    __syncthreads();
    // Exclusive scan of the counts: s_bend[b] = start of bucket b.  Up to 16
    // waves scan slices of 64 or more buckets, then add the totals of the
    // slices before theirs.
    {
      const int32_t nw = nb / kWave < kLocalWaves ? nb / kWave : kLocalWaves;
      const int32_t slice = nb / nw;
      int32_t carry = 0;
      if (wave < nw) {
        for (int32_t base = wave * slice; base < (wave + 1) * slice; base += kWave) {
          const int32_t v = s_bend[base + lane];
          const int32_t incl = wave_incl_scan(v);
          s_bend[base + lane] = carry + incl - v;
          carry += readlane(incl, kWave - 1);
        }
        if (lane == 0) s_slice_total[wave] = carry;
      }
      __syncthreads();
      if (wave > 0 && wave < nw) {
        int32_t before = 0;
        for (int32_t w = 0; w < wave; ++w) before += s_slice_total[w];
        for (int32_t base = wave * slice; base < (wave + 1) * slice; base += kWave) {
          s_bend[base + lane] += before;
        }
      }
    }
    __syncthreads();
    // 2a. Scatter: one thread per row writes its keys; the bucket cursor
    //     moves s_bend[b] from the start to the end of bucket b.  A thread
    //     reads its row in 16-byte groups (the aligned groups that cover the
    //     row, read whole only inside the chunk's nonzeros; a group at the
    //     chunk's edge is read element by element): the lanes of a wave read
    //     different rows, so each load instruction touches a line per lane,
    //     and a group's four columns cost one such access.  In tier 2, rows
    //     of more than kScatterRowCap nonzeros are scattered by the whole wave
    //     that holds them, 64 columns per load, after its other rows: on
    //     skewed graphs a thread per row left the step as long as the chunk's
    //     longest row.
    unsigned long long msum = 0; // this thread's rows' mirror-check terms, when asked
    const bool vec_ok = (reinterpret_cast<uintptr_t>(col_ind) & 15u) == 0;
    for (int32_t r0 = kWideRows ? wave * kWave : tid; r0 < rows;
         r0 += kLocalThreads) {
      const int32_t r = kWideRows ? r0 + lane : r0;
      const int32_t rb = (!kWideRows || r < rows) ? row_ptr[cs + r] : 0;
      const int32_t re = (!kWideRows || r < rows) ? rb + s_size[r] : 0;
      const bool wide = kWideRows && re - rb > kScatterRowCap;
      for (int32_t q = vec_ok ? (rb & ~3) : rb; !wide && q < re; q += vec_ok ? 4 : 1) {
        int32_t v[4];
        if (vec_ok && q >= e0 && q + 4 <= e0 + E) {
          const int4 g = *reinterpret_cast<const int4 *>(col_ind + q);
          v[0] = g.x;
          v[1] = g.y;
          v[2] = g.z;
          v[3] = g.w;
        } else {
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            v[u] = (q + u >= rb && q + u < re && (vec_ok || u == 0)) ? col_ind[q + u] : 0;
          }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (q + u >= rb && q + u < re && (vec_ok || u == 0)) {
            const uint32_t c = static_cast<uint32_t>(v[u]);
            const int32_t slot = atomicAdd(&s_bend[bucket_of(c, nbl)], 1);
            s_keys[slot] = (c << lb) | static_cast<uint32_t>(r);
            if (mirror != nullptr) msum += mirror_term(cs + r, static_cast<int32_t>(c));
          }
        }
      }
      if constexpr (kWideRows) {
        for (uint64_t wm = ballot(wide); wm != 0; wm = clear_bit(wm, __builtin_ctzll(wm))) {
          const int32_t i = __builtin_ctzll(wm);
          const int32_t wr = readlane(r, i), wb = readlane(rb, i), we = readlane(re, i);
          for (int32_t q = wb + lane; q < we; q += kWave) {
            const uint32_t c = static_cast<uint32_t>(col_ind[q]);
            const int32_t slot = atomicAdd(&s_bend[bucket_of(c, nbl)], 1);
            s_keys[slot] = (c << lb) | static_cast<uint32_t>(wr);
            if (mirror != nullptr) msum += mirror_term(cs + wr, static_cast<int32_t>(c));
          }
        }
      }
    }
    if (mirror != nullptr) {
      // One LDS atomic per wave: per-thread atomics on one LDS word serialise.
#pragma unroll
      for (int o = kWave / 2; o > 0; o >>= 1) msum += __shfl_xor(msum, o);
      if (lane == 0 && msum != 0) atomicAdd(&s_mirror, msum);
    }
    __syncthreads();
    // 2b. Sort each bucket: up to 16 keys by one thread in registers (a
    //     16-slot bitonic network), up to kSmallBucket by one thread in LDS
    //     (insertion sort) ...
    for (int32_t b0 = 0; b0 < nb; b0 += kLocalThreads) {
      const int32_t b = b0 + tid;
      const int32_t lo = (b < nb && b) ? s_bend[b - 1] : 0;
      const int32_t hi = b < nb ? s_bend[b] : 0;
      const int32_t sz = hi - lo;
      if (sz <= 16) {
        register_sort_keys<16>(s_keys, lo, sz);
      } else if (sz <= kSmallBucket) {
        for (int32_t i = lo + 1; i < hi; ++i) {
          const uint32_t x = s_keys[i];
          int32_t j = i - 1;
          while (j >= lo && s_keys[j] > x) {
            s_keys[j + 1] = s_keys[j];
            --j;
          }
          s_keys[j + 1] = x;
        }
      } else {
        // At most KEYCAP / (kSmallBucket + 1) such buckets: fits s_order.
        s_order[atomicAdd(&s_big_count, 1)] = static_cast<uint16_t>(b);
      }
    }
    __syncthreads();
    // ... large ones by one wave each, from the list.
    for (int32_t i = wave; i < s_big_count; i += kLocalWaves) {
      const int32_t b = s_order[i];
      const int32_t lo = b ? s_bend[b - 1] : 0, hi = s_bend[b];
      wave_sort_lds(s_keys + lo, hi - lo);
    }
    __syncthreads();

    // 3. Rows holding a column that another chunk row also holds (equal
    //    columns are adjacent now).
    for (int32_t i = tid; i < E; i += kLocalThreads) {
      const uint32_t key = s_keys[i];
      const uint32_t c = key >> lb;
      const bool multi = (i > 0 && (s_keys[i - 1] >> lb) == c) ||
                         (i + 1 < E && (s_keys[i + 1] >> lb) == c);
      if (multi) s_order[key & rmask] = kMultiMark;
    }
    __syncthreads();

    // 3b. Processing order: rows with candidates by floor(log2(row size)),
    //     largest first (a longest-first schedule with the row size standing
    //     in for the stream length), then the rows without candidates.  A
    //     counting sort; the order inside a class does not matter, since each
    //     row's table row depends on that row alone.
    int32_t my_class[kRowsPerThread];
#pragma unroll
    for (int u = 0; u < kRowsPerThread; ++u) {
      const int32_t r = tid + u * kLocalThreads;
      my_class[u] = -1;
      if (r < rows) {
        const int32_t sz = s_size[r];
        my_class[u] = (s_order[r] == kMultiMark && sz > 0) ? __clz(sz) : kClasses;
        atomicAdd(&s_class[my_class[u]], 1);
      }
    }
    __syncthreads();
    if (wave == 0) {
      const int32_t v = lane <= kClasses ? s_class[lane] : 0;
      const int32_t incl = wave_incl_scan(v);
      if (lane <= kClasses) s_class[lane] = incl - v;
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kRowsPerThread; ++u) {
      if (my_class[u] >= 0) {
        const int32_t r = tid + u * kLocalThreads;
        s_order[atomicAdd(&s_class[my_class[u]], 1)] = static_cast<uint16_t>(r);
      }
    }
    __syncthreads();

    // 4a. Rows without candidates (the tail of the order) get all-zero table
    //     rows from the whole workgroup, 16 lanes per row.
    const int32_t zero_start = s_class[kClasses - 1];
    for (int32_t zi = zero_start + tid / 16; zi < rows; zi += kLocalThreads / 16) {
      uint64_t *out = table + static_cast<size_t>(cs + s_order[zi]) * k;
      for (int32_t j = tid % 16; j < k; j += 16) out[j] = 0;
    }
    // 4b. Sketch, one wave per row.  Waves claim rows from a shared counter
    //     in the order of step 3b: stream lengths vary by orders of magnitude
    //     on skewed graphs, and a fixed row-to-wave assignment would leave the
    //     workgroup waiting on its most loaded wave.
    WaveSketch<CELLS> store;
    for (;;) {
      int32_t claim = 0;
      if (lane == 0) claim = atomicAdd(&s_next_row, 1);
      const int32_t idx = readlane(claim, 0);
      if (idx >= zero_start) break;
      const int32_t r = s_order[idx];
      const int32_t row = cs + r;
      uint64_t *out = table + static_cast<size_t>(row) * k;
      const int32_t row_size = s_size[r];
      store.clear();
      const int32_t rb = row_ptr[row], re = rb + row_size;
      for (int32_t pb = rb; pb < re; pb += kWave) {
        const int32_t p = pb + lane;
        int32_t a = 0, bnd = 0;
        if (p < re) {
          const uint32_t c = static_cast<uint32_t>(col_ind[p]);
          const uint32_t bk = bucket_of(c, nbl);
          const int32_t blo = bk ? s_bend[bk - 1] : 0, bhi = s_bend[bk];
          const uint32_t base = c << lb;
          a = lds_lower_bound(s_keys, blo, bhi, base);
          bnd = lds_upper_bound(s_keys, a, bhi, base | rmask);
        }
        const int32_t len = bnd - a;
        const int32_t incl = wave_incl_scan(len);
        const int32_t excl = incl - len;
        const int32_t total = readlane(incl, kWave - 1);
        for (int32_t f0 = 0; f0 < total; f0 += kWave) {
          const int32_t f = f0 + lane;
          int32_t j = 0;
#pragma unroll
          for (int step = 32; step > 0; step >>= 1) {
            const int32_t tt = j + step;
            const int32_t e = __shfl(excl, tt & (kWave - 1), kWave);
            if (tt < kWave && e <= f) j = tt;
          }
          const int32_t seg_a = __shfl(a, j, kWave);
          const int32_t seg_x = __shfl(excl, j, kWave);
          bool item = false;
          int32_t other = -1;
          float alpha = 0.0f;
          if (f < total) {
            const int32_t ol = static_cast<int32_t>(s_keys[seg_a + (f - seg_x)] & rmask);
            if (ol != r) {
              other = cs + ol;
              alpha = 2.0f / static_cast<float>(row_size + s_size[ol]);
              item = true;
            }
          }
          store.consume(ballot(item), other, alpha);
        }
      }
      store.select_top_k(k, out);
      if (row_valid != nullptr && lane == 0) row_valid[row] = min(k, store.filled);
    }
    __syncthreads(); // LDS is reused by the next chunk of this workgroup
  }
  // One global atomic per workgroup (the last barrier above ordered every
  // row's LDS atomic before this read).
  if (mirror != nullptr && threadIdx.x == 0 && s_mirror != 0) atomicAdd(mirror, s_mirror);
}

// Tier parameters: (key capacity, row capacity, log2 buckets).
constexpr int kT1Keys = 16384, kT1Rows = 1024, kT1Nb = 11;
constexpr int kT2Keys = 32768, kT2Rows = 4096, kT2Nb = 10;
// On a symmetric matrix the global path reads the CSR as its CSC (no
// transpose), and its waves, with little LDS, run on the CUs beside tier 2's
// one workgroup per CU: tier 2 then takes chunks of at most this many
// nonzeros and the larger ones go to the global path, which adds waves to
// the SIMDs that tier 2 leaves at four.  Measured on C5 (Chung-Lu, most
// chunks tier 2), csg median of 5, with the capacity-128 sketch update in
// GCN assembly: 36.7 ms with the split at 22528, 33.8 at 24576, 30.8 at
// 26624, 28.5 at 28672, 29.0 at 30720, 31.0 at 32768 (with the compiled
// update, whose tier-2 items cost more, 33.1 at 26624 was the best); C3
// unchanged.
constexpr int kT2SharedKeys = 28672;

constexpr int kClassifyThreads = 1024;
// Up to this many chunks one workgroup classifies and orders the lists,
// holding kClassifyPer chunk sizes per thread in registers.
constexpr int kClassifyPer = 8;
constexpr int kClassifyOrderCap = kClassifyThreads * kClassifyPer;

// Tier of a chunk of `rows` rows and E nonzeros: 1 and 2 are the LDS tiers
// (1 only when t1 is set), 3 the global-CSC path.  The tier-1 test and the
// capacities are the tier kernels' own; t2_keys (at most kT2Keys) is where
// tier 2 hands chunks to the global path.
__device__ __forceinline__ int chunk_tier(int32_t E, int32_t rows, bool t1, int32_t t2_keys) {
  if (t1 && E <= kT1Keys && rows <= kT1Rows) return 1;
  if (E <= t2_keys && rows <= kT2Rows) return 2;
  return 3;
}

// List of a chunk of tier t: 0 for tier 2, 1 for the global path, 2 for
// tier 1 (-1: none).
__device__ __forceinline__ int tier_list(int tier) {
  return tier == 1 ? 2 : (tier >= 2 ? tier - 2 : -1);
}

// Lists the chunks by tier: tier-2 chunks in lists[0 .. counts[0]),
// global-path chunks in lists[chunks .. chunks + counts[1]), tier-1 chunks in
// lists[2 chunks .. 2 chunks + counts[2]); counts[3] = 0 (the counter tier 2
// claims its chunks from).  With one workgroup the tier-2 and global lists
// are ordered by floor(log2(nonzeros)), largest first (a counting sort in
// LDS; order inside a class is arbitrary), so heavy chunks start first; the
// tier-1 list is unordered (one LDS atomic per wave: on inputs of many
// similar chunks a counting sort put them all on one class counter); and
// counts are written, not added.  With several workgroups (more than kClassifyOrderCap
// chunks) the lists are unordered and counts must be zero on entry.  The
// table does not depend on list order.
__global__ void __launch_bounds__(kClassifyThreads)
    classify_chunks_kernel(int32_t n, int32_t chunk_size, int t1, int32_t t2_keys,
                           const int32_t *__restrict__ row_ptr, int32_t *__restrict__ lists,
                           int32_t *__restrict__ counts) {
  __shared__ int32_t s_cls[2][kClasses + 1];
  __shared__ int32_t s_t1;
  const int64_t chunks = ceil_div64(n, chunk_size);
  const int tid = threadIdx.x, lane = lane_id();
  auto chunk_of = [&](int64_t q, int32_t *E) {
    const int64_t cs = q * chunk_size;
    const int64_t ce = cs + chunk_size < n ? cs + chunk_size : n;
    *E = row_ptr[ce] - row_ptr[cs];
    return chunk_tier(*E, static_cast<int32_t>(ce - cs), t1 != 0, t2_keys);
  };
  if (gridDim.x > 1) {
    for (int64_t q0 = static_cast<int64_t>(blockIdx.x) * kClassifyThreads; q0 < chunks;
         q0 += static_cast<int64_t>(gridDim.x) * kClassifyThreads) {
      const int64_t q = q0 + tid;
      int32_t E = 0;
      const int li = q < chunks ? tier_list(chunk_of(q, &E)) : -1;
#pragma unroll
      for (int l = 0; l < 3; ++l) {
        const uint64_t m = ballot(li == l);
        int32_t base = 0;
        if (m != 0 && lane == 0) base = atomicAdd(&counts[l], __popcll(m));
        base = readlane(base, 0);
        if (li == l) {
          lists[l * chunks + base + __popcll(m & ((1ull << lane) - 1ull))] =
              static_cast<int32_t>(q);
        }
      }
    }
    return;
  }
  for (int i = tid; i < 2 * (kClasses + 1); i += kClassifyThreads) (&s_cls[0][0])[i] = 0;
  if (tid == 0) {
    s_t1 = 0;
    counts[3] = 0;
  }
  // Chunk tid + u * kClassifyThreads: its list and its class 31 -
  // floor(log2(E)) (ascending class = descending size).
  int li[kClassifyPer], cls[kClassifyPer];
#pragma unroll
  for (int u = 0; u < kClassifyPer; ++u) {
    const int64_t q = tid + static_cast<int64_t>(u) * kClassifyThreads;
    int32_t E = 0;
    li[u] = q < chunks ? tier_list(chunk_of(q, &E)) : -1;
    cls[u] = __clz(E > 0 ? E : 1);
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kClassifyPer; ++u) {
    if (li[u] == 0 || li[u] == 1) atomicAdd(&s_cls[li[u]][cls[u]], 1);
    const uint64_t m = ballot(li[u] == 2);
    int32_t base = 0;
    if (m != 0 && lane == 0) base = atomicAdd(&s_t1, __popcll(m));
    base = readlane(base, 0);
    if (li[u] == 2) {
      lists[2 * chunks + base + __popcll(m & ((1ull << lane) - 1ull))] =
          tid + u * kClassifyThreads;
    }
  }
  __syncthreads();
  if (tid == 2) counts[2] = s_t1;
  if (tid < 2) {
    int32_t run = 0;
    for (int c = 0; c <= kClasses; ++c) {
      const int32_t v = s_cls[tid][c];
      s_cls[tid][c] = run;
      run += v;
    }
    counts[tid] = run;
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kClassifyPer; ++u) {
    if (li[u] == 0 || li[u] == 1) {
      const int l = li[u];
      lists[l * chunks + atomicAdd(&s_cls[l][cls[u]], 1)] =
          tid + u * kClassifyThreads;
    }
  }
}

template <int CELLS, int KEYCAP, int ROWCAP, int NB_LOG2, bool CLAIM>
void launch_tier(Context &ctx, int32_t n, int32_t k, int32_t chunk_size, int32_t lb,
                 const int32_t *d_ptr, const int32_t *d_ind, uint64_t *d_table,
                 const int32_t *list, const int32_t *list_count, int64_t host_len,
                 int32_t *ovf, int32_t *ovf_count, int per_cu, int32_t *d_row_valid,
                 unsigned long long *mirror, uint32_t *claim) {
  const int64_t chunks = ceil_div64(n, chunk_size);
  // A fixed grid striding over (or claiming from) the work: no launch per
  // chunk of an empty list, and with the list's length known on the host, no
  // more workgroups than entries.
  const int64_t len = host_len >= 0 ? std::min<int64_t>(host_len, chunks) : chunks;
  const int64_t grid =
      list ? std::min<int64_t>(len, static_cast<int64_t>(ctx.num_cus) * per_cu) : chunks;
  if (grid <= 0) return;
  chunk_local_sketch_kernel<CELLS, KEYCAP, ROWCAP, NB_LOG2, CLAIM>
      <<<dim3(static_cast<unsigned>(grid)), kLocalThreads, 0, ctx.stream>>>(
          n, k, chunk_size, lb, d_ptr, d_ind, d_table, list, list_count, ovf, ovf_count,
          d_row_valid, mirror, claim);
  SP_LAUNCH_CHECK();
}

template <int CELLS>
void launch_local(Context &ctx, int32_t n, int32_t k, int32_t chunk_size, int32_t lb,
                  const int32_t *d_ptr, const int32_t *d_ind, uint64_t *d_table,
                  const int32_t *lists, int32_t *counts, int tiers, int64_t t1_list_len,
                  int32_t *d_row_valid, unsigned long long *mirror) {
  const int64_t chunks = ceil_div64(n, chunk_size);
  if (tiers & 2) {
    launch_tier<CELLS, kT2Keys, kT2Rows, kT2Nb, true>(
        ctx, n, k, chunk_size, lb, d_ptr, d_ind, d_table, lists, counts, -1, nullptr, nullptr,
        1, d_row_valid, mirror, reinterpret_cast<uint32_t *>(counts + 3));
  }
  if ((tiers & 1) && chunk_size <= kT1Rows) {
    const bool listed = t1_list_len >= 0;
    launch_tier<CELLS, kT1Keys, kT1Rows, kT1Nb, false>(
        ctx, n, k, chunk_size, lb, d_ptr, d_ind, d_table, listed ? lists + 2 * chunks : nullptr,
        listed ? counts + 2 : nullptr, t1_list_len, nullptr, nullptr, 2, d_row_valid, mirror,
        nullptr);
  }
}

} // namespace

bool chunk_local_supported(int32_t n, int32_t chunk_size) {
  return chunk_size <= kLocalRowCap && bits_for(n - 1) + bits_for(chunk_size - 1) <= 32;
}

void chunk_local_classify(Context &ctx, int32_t n, int32_t chunk_size, const int32_t *d_ptr,
                          int32_t *d_lists, int32_t *d_counts, bool is_symmetric) {
  SP_EXPECT(chunk_local_supported(n, chunk_size), "chunk-local sketch not applicable");
  const int64_t chunks = ceil_div64(n, chunk_size);
  const int t1 = chunk_size <= kT1Rows ? 1 : 0;
  int grid = 1;
  if (chunks > kClassifyOrderCap) {
    grid = ctx.grid_for(ceil_div64(chunks, kClassifyThreads), kClassifyThreads, 1);
    fill_u32(ctx, d_counts, 4, 0u);
  }
  const int32_t t2_keys = is_symmetric ? kT2SharedKeys : kT2Keys;
  classify_chunks_kernel<<<grid, kClassifyThreads, 0, ctx.stream>>>(n, chunk_size, t1, t2_keys,
                                                                    d_ptr, d_lists, d_counts);
  SP_LAUNCH_CHECK();
}

void chunk_local_sketch_top_k(Context &ctx, int32_t n, int32_t k, int32_t chunk_size,
                              int32_t m_capacity, const int32_t *d_ptr, const int32_t *d_ind,
                              uint64_t *d_table, const int32_t *d_lists,
                              int32_t *d_counts, int tiers, int32_t *d_row_valid,
                              unsigned long long *mirror, int64_t t1_list_len) {
  SP_EXPECT(k <= 512, "k must be <= 512");
  SP_EXPECT(chunk_local_supported(n, chunk_size), "chunk-local sketch not applicable");
  const int32_t lb = bits_for(chunk_size - 1);
  switch (m_capacity / 32) {
#define SP_CASE(C)                                                                       \
  case C:                                                                                \
    launch_local<C>(ctx, n, k, chunk_size, lb, d_ptr, d_ind, d_table, d_lists, d_counts, \
                    tiers, t1_list_len, d_row_valid, mirror);                            \
    break;
    SP_CASE(1) SP_CASE(2) SP_CASE(3) SP_CASE(4) SP_CASE(5) SP_CASE(6)
    SP_CASE(7) SP_CASE(8) SP_CASE(9) SP_CASE(10) SP_CASE(11) SP_CASE(12)
    SP_CASE(13) SP_CASE(14) SP_CASE(15) SP_CASE(16)
#undef SP_CASE
  default:
    SP_EXPECT(false, "sketch capacity must be a multiple of 32 in [32, 512]");
  }
}

} // namespace sporder_hip
