// csg_overflow.hip -- sketch + top-k from the global CSC, for the rows of
// chunks the LDS tiers cannot hold (and for every row when the chunk-local
// path does not apply, e.g. the one-chunk global sketch).
//
// The CSC is the transpose, or the CSR itself when is_symmetric
// (sporder/src/common/csr2csc.h:49-59).  Row r's candidate stream
// (sporder/src/common/chunk_similarity_top_k.cu:53-83): for each column c of r
// in CSR order, the rows s of column c in ascending order with
// cs <= s < ce and s != r, each with weight fl(2 / (float)(|r| + |s|)).  The
// rows of column c inside [cs, ce) are one contiguous run of the CSC column,
// so the stream is the concatenation of one run per nonzero of r.
//
// Four launches:
//   1. plan (one workgroup): the listed chunks' nonzeros cut into tasks of
//      kRunTask; exclusive task offsets per list entry.
//   2. pairs (one lane per CSC entry): (row, |row|), so one 8-byte load gives
//      an item's key and the operand of its weight; and every 16th CSC row
//      index copied into a sample (nnz/16 words) for the run search.
//   3. runs (one lane per nonzero of the listed chunks): the run [a, a + len)
//      of the chunk's rows in the nonzero's column, by a binary search over
//      the sample finished inside one 64-byte line, then a gallop.  The
//      searches of one row are spread over the whole device, so a hub row
//      with 600K columns costs 600K independent searches, not one wave's
//      serial walk.
//   4. sketch (one wave per row): walks the row's runs 64 nonzeros at a time
//      with four blocks of runs in flight and item batches loaded one batch
//      ahead, feeding the wave64 space-saving sketch (sketch.hpp).  An item's
//      run is found by marking run starts in LDS and a DPP running maximum.
// The stream, and therefore the table, is the reference's.
#include "common.hpp"
#include "sketch.hpp"

namespace sporder_hip {

namespace {

constexpr int kRunTask = 1024;   // nonzeros per runs task
// One workgroup of 4 waves: small enough to be placed beside an LDS tier-2
// workgroup, which leaves a CU too few wave slots for a 16-wave group.
constexpr int kPlanBlock = 256;
constexpr int kRunsBlock = 256;
constexpr int kOvfBlock = 256;
constexpr int kOvfWaves = kOvfBlock / kWave;
constexpr int kMirrorBlock = 256;
constexpr int kMirrorRowCap = 64; // longer rows: the whole wave (ovf_mirror_kernel)
constexpr int kSample = 16;      // run-search sample stride (one 64-byte line)

__device__ __forceinline__ int64_t list_len(const int32_t *list, const int32_t *list_count,
                                            int64_t num_chunks) {
  return list ? static_cast<int64_t>(*list_count) : num_chunks;
}

// List entries [l0, l1) of a launch; l1 < 0: to the end of the list.
__device__ __forceinline__ int64_t range_end(int64_t l1, const int32_t *list,
                                             const int32_t *list_count, int64_t num_chunks) {
  const int64_t L = list_len(list, list_count, num_chunks);
  return l1 < 0 || l1 > L ? L : l1;
}

// task_off[i] = tasks of list entries before i; task_off[L] = total.
__global__ void __launch_bounds__(kPlanBlock)
    ovf_plan_kernel(int32_t n, int32_t chunk_size, const int32_t *__restrict__ row_ptr,
                    const int32_t *__restrict__ list, const int32_t *__restrict__ list_count,
                    int32_t *__restrict__ task_off) {
  __shared__ int32_t wave_tot[kPlanBlock / kWave];
  __shared__ int32_t s_carry;
  const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
  const int64_t L = list_len(list, list_count, ceil_div64(n, chunk_size));
  if (tid == 0) s_carry = 0;
  __syncthreads();
  for (int64_t base = 0; base < L; base += kPlanBlock) {
    const int64_t i = base + tid;
    int32_t v = 0;
    if (i < L) {
      const int64_t q = list ? list[i] : i;
      const int64_t cs = q * chunk_size;
      const int64_t ce = cs + chunk_size < n ? cs + chunk_size : n;
      v = static_cast<int32_t>(ceil_div64(row_ptr[ce] - row_ptr[cs], kRunTask));
    }
    const int32_t incl = wave_incl_scan(v);
    if (lane == kWave - 1) wave_tot[wave] = incl;
    __syncthreads();
    int32_t before = s_carry, all = 0;
#pragma unroll
    for (int w = 0; w < kPlanBlock / kWave; ++w) {
      const int32_t t = wave_tot[w];
      before += (w < wave) ? t : 0;
      all += t;
    }
    if (i < L) task_off[i] = before + incl - v;
    __syncthreads();
    if (tid == 0) s_carry += all;
    __syncthreads();
  }
  if (tid == 0) task_off[L] = s_carry;
}

// First index in [lo, hi) with a[i] >= t, for a sorted range of `a` whose
// every kSample-th element (global positions 0, kSample, 2*kSample, ...) is
// copied in `sample`: the search runs over the sample, a small array that
// stays in cache, and ends inside one 64-byte line of `a`.
__device__ __forceinline__ int32_t sampled_lower_bound(const int32_t *__restrict__ a,
                                                       const int32_t *__restrict__ sample,
                                                       int32_t lo, int32_t hi, int32_t t) {
  if (hi - lo < 2 * kSample) return lower_bound_dev(a, lo, hi, t);
  // Samples at positions inside [lo, hi): indices [s_lo, s_hi).
  const int32_t s_lo = (lo + kSample - 1) / kSample, s_hi = (hi - 1) / kSample + 1;
  const int32_t s = lower_bound_dev(sample, s_lo, s_hi, t);
  // a[kSample*(s-1)] < t (when s > s_lo) and a[kSample*s] >= t (when s < s_hi).
  const int32_t from = s > s_lo ? kSample * (s - 1) + 1 : lo;
  const int32_t to = s < s_hi ? kSample * s : hi;
  return lower_bound_dev(a, from, to, t);
}

// Runs of the nonzeros of list entries [l0, l1) (l1 < 0: to the end).
__global__ void __launch_bounds__(kRunsBlock)
    ovf_runs_kernel(int32_t n, int32_t chunk_size, const int32_t *__restrict__ row_ptr,
                    const int32_t *__restrict__ col_ind, const int32_t *__restrict__ col_ptr,
                    const int32_t *__restrict__ row_ind, const int32_t *__restrict__ sample,
                    const int32_t *__restrict__ list, const int32_t *__restrict__ list_count,
                    const int32_t *__restrict__ task_off, int2 *__restrict__ runs, int64_t l0,
                    int64_t l1) {
  const int64_t L = range_end(l1, list, list_count, ceil_div64(n, chunk_size));
  if (L <= l0) return;
  const int32_t tasks = task_off[L];
  for (int32_t t = task_off[l0] + blockIdx.x; t < tasks; t += gridDim.x) {
    // List entry owning task t: the largest i with task_off[i] <= t (entries
    // without tasks share their successor's offset and are skipped).
    int64_t lo = l0, hi = L - 1;
    while (lo < hi) {
      const int64_t mid = (lo + hi + 1) >> 1;
      if (task_off[mid] <= t) {
        lo = mid;
      } else {
        hi = mid - 1;
      }
    }
    const int64_t q = list ? list[lo] : lo;
    const int64_t cs64 = q * chunk_size;
    const int32_t cs = static_cast<int32_t>(cs64);
    const int32_t ce = static_cast<int32_t>(cs64 + chunk_size < n ? cs64 + chunk_size : n);
    const int64_t e1 = row_ptr[ce];
    const int64_t p0 = row_ptr[cs] + static_cast<int64_t>(t - task_off[lo]) * kRunTask;
    const int64_t p1 = p0 + kRunTask < e1 ? p0 + kRunTask : e1;
    for (int64_t p = p0 + threadIdx.x; p < p1; p += kRunsBlock) {
      const int32_t c = col_ind[p];
      const int32_t b0 = col_ptr[c], b1 = col_ptr[c + 1];
      const int32_t a = sampled_lower_bound(row_ind, sample, b0, b1, cs);
      // The run of chunk rows is short next to the column: gallop from a.
      const int32_t b = gallop_lower_bound(row_ind, a, b1, ce);
      runs[p] = make_int2(a, b - a);
    }
  }
}

// pairs[t] = (row, |row|) of CSC entry t, and the run search's sample of
// every kSample-th entry.
__global__ void __launch_bounds__(256)
    ovf_pairs_kernel(int32_t nnz, const int32_t *__restrict__ row_ptr,
                     const int32_t *__restrict__ row_ind, const int32_t *__restrict__ list,
                     const int32_t *__restrict__ list_count, int2 *__restrict__ pairs,
                     int32_t *__restrict__ sample) {
  if (list && *list_count == 0) return;
  for (int64_t t = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; t < nnz;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int32_t s = row_ind[t];
    pairs[t] = make_int2(s, row_ptr[s + 1] - row_ptr[s]);
    if (t % kSample == 0) sample[t / kSample] = s;
  }
}

// Runs of nonzeros [rs + 64*blk, +64) of the row.  The load is issued by
// every lane (an index past the row reads the row's last run and the caller
// masks it), so the compiler can keep several of these in flight: a load under
// a branch makes the next wait count drain the whole queue.
__device__ __forceinline__ int2 load_runs(const int2 *__restrict__ runs, int32_t rs,
                                          int32_t re, int32_t blk, int lane) {
  const int64_t p = static_cast<int64_t>(rs) + static_cast<int64_t>(blk) * kWave + lane;
  return runs[p < re ? p : re - 1];
}

// Per-wave LDS scratch of the item-to-run lookup.
struct RunLookup {
  int32_t mark[kWave]; // run index + 1 starting at each item slot of a batch
  int32_t base[kWave]; // a_j - excl_j: CSC index of item f is base[j] + f
};

// CSC indices of items f0 .. f0+63 of a block whose run j (lane j) starts at
// item excl_j and holds len_j items.  Each run starting inside the batch marks
// its first slot with j + 1; a running maximum carries the run over its items
// (`carry` is the run, + 1, of item f0 - 1 and is updated).  Lanes past the
// block's total return index 0 (a valid address; the caller masks them).
// Every lane must be active.
__device__ __forceinline__ int32_t item_index(RunLookup *lk, int32_t len, int32_t excl,
                                              int32_t total, int32_t f0, int32_t *carry,
                                              int lane) {
  const int32_t rel = excl - f0;
  lk->mark[lane] = 0;
  wave_lds_order();
  if (len > 0 && rel >= 0 && rel < kWave) lk->mark[rel] = lane + 1;
  wave_lds_order();
  int32_t m = lk->mark[lane];
  if (lane == 0 && m == 0) m = *carry;
  m = wave_incl_max(m);
  *carry = readlane(m, kWave - 1);
  const int32_t f = f0 + lane;
  const int32_t t = lk->base[m - 1] + f;
  return f < total ? t : 0;
}

template <int CELLS>
__device__ __forceinline__ void feed_batch(WaveSketch<CELLS> &store, int2 pr, int32_t f0,
                                           int32_t total, int32_t row, int32_t deg,
                                           int lane) {
  const bool item = f0 + lane < total && pr.x != row;
  const float alpha = 2.0f / static_cast<float>(deg + pr.y);
  store.feed(ballot(item), pr.x, alpha);
}

// One block of 64 runs through the sketch, item batches two at a time with
// the second batch's load in flight while the first is applied.
template <int CELLS>
__device__ __forceinline__ void feed_block(WaveSketch<CELLS> &store, RunLookup *lk,
                                           const int2 *__restrict__ pairs, int2 run,
                                           bool in_row, int32_t row, int32_t deg, int lane) {
  const int32_t a = run.x;
  const int32_t len = in_row ? run.y : 0;
  const int32_t incl = wave_incl_scan(len);
  const int32_t excl = incl - len;
  const int32_t total = readlane(incl, kWave - 1);
  if (total == 0) return;
  lk->base[lane] = a - excl;
  int32_t carry = 0;
  int2 b0 = pairs[item_index(lk, len, excl, total, 0, &carry, lane)];
  for (int32_t f0 = 0; f0 < total; f0 += 2 * kWave) {
    const int2 b1 = pairs[item_index(lk, len, excl, total, f0 + kWave, &carry, lane)];
    // Keep the scheduler from hoisting b0's first use above b1's load: the
    // wait for b0 must leave b1 in flight.
    __builtin_amdgcn_sched_barrier(0);
    feed_batch(store, b0, f0, total, row, deg, lane);
    b0 = pairs[item_index(lk, len, excl, total, f0 + 2 * kWave, &carry, lane)];
    __builtin_amdgcn_sched_barrier(0);
    if (f0 + kWave < total) feed_batch(store, b1, f0 + kWave, total, row, deg, lane);
  }
}

template <int CELLS>
__global__ void __launch_bounds__(kOvfBlock)
    ovf_sketch_kernel(int32_t n, int32_t k, int32_t chunk_size,
                      const int32_t *__restrict__ row_ptr, const int2 *__restrict__ runs,
                      const int2 *__restrict__ pairs, uint64_t *__restrict__ table,
                      const int32_t *__restrict__ list,
                      const int32_t *__restrict__ list_count, uint32_t *__restrict__ claim,
                      int32_t *__restrict__ row_valid, int64_t l0, int64_t l1) {
  __shared__ RunLookup s_lookup[kOvfWaves];
  const int lane = lane_id();
  RunLookup *lk = &s_lookup[threadIdx.x / kWave];
  // Rows of list entries [l0, l1); work < 2^32: list_len * chunk_size <=
  // n + chunk_size - 1.
  const int64_t L = range_end(l1, list, list_count, ceil_div64(n, chunk_size));
  const int64_t work = (L > l0 ? L - l0 : 0) * chunk_size;
  WaveSketch<CELLS> store;

  // Waves claim rows one at a time from a device-wide counter (zeroed by the
  // host before the launch): a few rows stream millions of items, and a
  // fixed assignment would give one wave several of them.
  for (;;) {
    uint32_t claimed = 0;
    if (lane == 0) claimed = atomicAdd(claim, 1u);
    const int64_t w = static_cast<uint32_t>(readlane(static_cast<int32_t>(claimed), 0));
    if (w >= work) break;
    int64_t row64 = l0 * chunk_size + w;
    if (list) {
      row64 = static_cast<int64_t>(list[l0 + w / chunk_size]) * chunk_size + (w % chunk_size);
    }
    if (row64 >= n) continue;
    const int32_t row = static_cast<int32_t>(row64);
    uint64_t *out = table + static_cast<size_t>(row) * k;
    const int32_t rs = row_ptr[row], re = row_ptr[row + 1];
    const int32_t deg = re - rs;
    if (deg == 0) {
      for (int32_t j = lane; j < k; j += kWave) out[j] = 0;
      if (row_valid != nullptr && lane == 0) row_valid[row] = 0;
      continue;
    }
    store.clear();
    const int32_t nblk = (deg + kWave - 1) / kWave;
    // Four blocks of runs in flight, each in its own registers (a rotating
    // copy would wait for the loads it copies).
    int2 r0 = load_runs(runs, rs, re, 0, lane);
    int2 r1 = load_runs(runs, rs, re, 1, lane);
    int2 r2 = load_runs(runs, rs, re, 2, lane);
    int2 r3 = load_runs(runs, rs, re, 3, lane);
    for (int32_t blk = 0; blk < nblk; blk += 4) {
      const int64_t p = static_cast<int64_t>(rs) + static_cast<int64_t>(blk) * kWave + lane;
      feed_block(store, lk, pairs, r0, p < re, row, deg, lane);
      r0 = load_runs(runs, rs, re, blk + 4, lane);
      if (blk + 1 >= nblk) break;
      feed_block(store, lk, pairs, r1, p + kWave < re, row, deg, lane);
      r1 = load_runs(runs, rs, re, blk + 5, lane);
      if (blk + 2 >= nblk) break;
      feed_block(store, lk, pairs, r2, p + 2 * kWave < re, row, deg, lane);
      r2 = load_runs(runs, rs, re, blk + 6, lane);
      if (blk + 3 >= nblk) break;
      feed_block(store, lk, pairs, r3, p + 3 * kWave < re, row, deg, lane);
      r3 = load_runs(runs, rs, re, blk + 7, lane);
    }
    store.select_top_k(k, out);
    if (row_valid != nullptr && lane == 0) row_valid[row] = min(k, store.filled);
  }
}

// The is_symmetric mirror check of the listed chunks' rows: mirror_term
// (common.hpp) of every nonzero, summed into *mirror.  A wave takes 64
// consecutive rows, a lane per row of at most kMirrorRowCap nonzeros (four
// column loads in flight per lane), then its longer rows one by one with all
// lanes.  Kept out of the sketch kernel, where each row waited out its column
// loads before its sketch could start.
__global__ void __launch_bounds__(kMirrorBlock)
    ovf_mirror_kernel(int32_t n, int32_t chunk_size, const int32_t *__restrict__ row_ptr,
                      const int32_t *__restrict__ col_ind, const int32_t *__restrict__ list,
                      const int32_t *__restrict__ list_count,
                      unsigned long long *__restrict__ mirror) {
  __shared__ unsigned long long s_sum;
  if (threadIdx.x == 0) s_sum = 0;
  __syncthreads();
  const int lane = lane_id();
  constexpr int kWaves = kMirrorBlock / kWave;
  // Row slots of the listed chunks, taken 64 at a time (chunk_size need not
  // be a multiple of 64: a group may span two chunks).
  const int64_t work = list_len(list, list_count, ceil_div64(n, chunk_size)) * chunk_size;
  unsigned long long msum = 0;
  for (int64_t g = (static_cast<int64_t>(blockIdx.x) * kWaves + threadIdx.x / kWave) * kWave;
       g < work; g += static_cast<int64_t>(gridDim.x) * kWaves * kWave) {
    const int64_t w = g + lane;
    int32_t row = -1, rs = 0, re = 0;
    if (w < work) {
      const int64_t row64 =
          list ? static_cast<int64_t>(list[w / chunk_size]) * chunk_size + w % chunk_size : w;
      if (row64 < n) {
        row = static_cast<int32_t>(row64);
        rs = row_ptr[row];
        re = row_ptr[row + 1];
      }
    }
    const bool wide = re - rs > kMirrorRowCap;
    for (int32_t q0 = rs; !wide && q0 < re; q0 += 4) {
      int32_t c[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) c[u] = q0 + u < re ? col_ind[q0 + u] : 0;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (q0 + u < re) msum += mirror_term(row, c[u]);
      }
    }
    for (uint64_t wm = ballot(wide); wm != 0; wm = clear_bit(wm, __builtin_ctzll(wm))) {
      const int i = __builtin_ctzll(wm);
      const int32_t wr = readlane(row, i), wb = readlane(rs, i), we = readlane(re, i);
      for (int32_t q0 = wb; q0 < we; q0 += 4 * kWave) {
        int32_t c[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int32_t q = q0 + u * kWave + lane;
          c[u] = q < we ? col_ind[q] : 0;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (q0 + u * kWave + lane < we) msum += mirror_term(wr, c[u]);
        }
      }
    }
  }
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) msum += __shfl_xor(msum, o);
  if (lane == 0 && msum != 0) atomicAdd(&s_sum, msum);
  __syncthreads();
  if (threadIdx.x == 0 && s_sum != 0) atomicAdd(mirror, s_sum);
}

template <int CELLS>
void launch_ovf_sketch(Context &ctx, int32_t n, int32_t k, int32_t chunk_size,
                       const int32_t *d_ptr, const int2 *runs, const int2 *pairs,
                       uint64_t *d_table, const int32_t *list, const int32_t *list_count,
                       uint32_t *claim, int32_t *d_row_valid, int64_t l0, int64_t l1,
                       int64_t rows) {
  // A wave per row at most: rows = the launch's row slots when the host knows
  // them (a grid sized for every row of the matrix made a one-chunk launch
  // dispatch thousands of workgroups that found no row, holding back the
  // kernels queued beside it).
  const int g = ctx.grid_for(ceil_div64(rows >= 0 ? rows : n, kOvfWaves), kOvfBlock, 4);
  fill_u32(ctx, claim, 1, 0u);
  ovf_sketch_kernel<CELLS><<<g, kOvfBlock, 0, ctx.stream>>>(n, k, chunk_size, d_ptr, runs,
                                                            pairs, d_table, list, list_count,
                                                            claim, d_row_valid, l0, l1);
  SP_LAUNCH_CHECK();
}

} // namespace

void chunk_mirror_check(Context &ctx, int32_t n, int32_t chunk_size, const int32_t *d_ptr,
                        const int32_t *d_ind, const int32_t *d_chunks,
                        const int32_t *d_chunk_count, int64_t host_list_len,
                        unsigned long long *mirror) {
  const int64_t rows_bound =
      d_chunks == nullptr ? n : (host_list_len >= 0 ? host_list_len * chunk_size : n);
  if (rows_bound <= 0) return;
  const int gm = ctx.grid_for(ceil_div64(rows_bound, kMirrorBlock), kMirrorBlock, 2);
  ovf_mirror_kernel<<<gm, kMirrorBlock, 0, ctx.stream>>>(n, chunk_size, d_ptr, d_ind, d_chunks,
                                                          d_chunk_count, mirror);
  SP_LAUNCH_CHECK();
}

size_t chunk_sketch_ws_bytes(int32_t n, int32_t nnz, int32_t chunk_size) {
  return 2 * ws_bytes<int2>(static_cast<size_t>(nnz)) +
         ws_bytes<int32_t>(static_cast<size_t>(ceil_div64(n, chunk_size)) + 1) +
         ws_bytes<uint32_t>(2) + ws_bytes<int32_t>(static_cast<size_t>(nnz) / kSample + 1);
}

void chunk_sketch_top_k(Context &ctx, int32_t n, int32_t nnz, int32_t k, int32_t chunk_size,
                        int32_t m_capacity, const int32_t *d_ptr, const int32_t *d_ind,
                        const int32_t *d_col_ptr, const int32_t *d_row_ind,
                        uint64_t *d_table, const int32_t *d_chunks,
                        const int32_t *d_chunk_count, hipEvent_t prepared,
                        int32_t *d_row_valid, int64_t host_list_len) {
  SP_EXPECT(k <= 512, "k must be <= 512");
  SP_EXPECT(m_capacity % 32 == 0 && m_capacity >= 32 && m_capacity <= 512,
            "sketch capacity must be a multiple of 32 in [32, 512]");
  const int64_t chunks = ceil_div64(n, chunk_size);
  int2 *runs = ctx.take<int2>(static_cast<size_t>(nnz));
  int2 *pairs = ctx.take<int2>(static_cast<size_t>(nnz));
  int32_t *task_off = ctx.take<int32_t>(static_cast<size_t>(chunks) + 1);
  uint32_t *claim = ctx.take<uint32_t>(2);
  int32_t *sample = ctx.take<int32_t>(static_cast<size_t>(nnz) / kSample + 1);

  ovf_plan_kernel<<<1, kPlanBlock, 0, ctx.stream>>>(n, chunk_size, d_ptr, d_chunks,
                                                    d_chunk_count, task_off);
  SP_LAUNCH_CHECK();
  const int gp = ctx.grid_for(ceil_div64(nnz, 256), 256, 4);
  ovf_pairs_kernel<<<gp, 256, 0, ctx.stream>>>(nnz, d_ptr, d_row_ind, d_chunks,
                                               d_chunk_count, pairs, sample);
  SP_LAUNCH_CHECK();
  const int64_t max_tasks = ceil_div64(nnz, kRunTask) + chunks;
  const int gr = ctx.grid_for(max_tasks, kRunsBlock, 4);
  auto runs_launch = [&](int64_t l0, int64_t l1) {
    ovf_runs_kernel<<<gr, kRunsBlock, 0, ctx.stream>>>(n, chunk_size, d_ptr, d_ind, d_col_ptr,
                                                       d_row_ind, sample, d_chunks,
                                                       d_chunk_count, task_off, runs, l0, l1);
    SP_LAUNCH_CHECK();
  };
  auto sketch_launch = [&](uint32_t *cl, int64_t l0, int64_t l1) {
    // Row slots of list entries [l0, l1) when the list's length is known.
    int64_t rows = -1;
    if (d_chunks == nullptr) {
      rows = n;
    } else if (host_list_len >= 0) {
      const int64_t e = l1 < 0 || l1 > host_list_len ? host_list_len : l1;
      rows = (e > l0 ? e - l0 : 0) * chunk_size;
    }
    switch (m_capacity / 32) {
#define SP_CASE(C)                                                                         \
  case C:                                                                                  \
    launch_ovf_sketch<C>(ctx, n, k, chunk_size, d_ptr, runs, pairs, d_table, d_chunks,     \
                         d_chunk_count, cl, d_row_valid, l0, l1, rows);                    \
    break;
      SP_CASE(1) SP_CASE(2) SP_CASE(3) SP_CASE(4) SP_CASE(5) SP_CASE(6)
      SP_CASE(7) SP_CASE(8) SP_CASE(9) SP_CASE(10) SP_CASE(11) SP_CASE(12)
      SP_CASE(13) SP_CASE(14) SP_CASE(15) SP_CASE(16)
#undef SP_CASE
    default:
      break;
    }
  };
  if (d_chunks == nullptr || host_list_len < 2) {
    runs_launch(0, -1);
    if (prepared != nullptr) SP_HIP(hipEventRecord(prepared, ctx.stream));
    sketch_launch(claim, 0, -1);
    return;
  }
  // The first listed chunk (the largest size class; on power-law inputs it
  // holds the hub rows whose serial sketch chains are the critical path) has
  // its run search alone, then its sketch on this stream while the other
  // chunks' run search and sketch run beside it on side stream 2.  Measured
  // on C3: the full run search takes 17 ms, which the hub rows' chain no
  // longer waits for; run beside the other chunks' search, the first chunk's
  // took 13 ms.
  runs_launch(0, 1);
  fork_side(ctx, 2);
  sketch_launch(claim, 0, 1);
  {
    OnStream on(ctx, ctx.side[2]);
    runs_launch(1, -1);
    if (prepared != nullptr) SP_HIP(hipEventRecord(prepared, ctx.stream));
    sketch_launch(claim + 1, 1, -1);
  }
  join_side(ctx, 2);
}

} // namespace sporder_hip
