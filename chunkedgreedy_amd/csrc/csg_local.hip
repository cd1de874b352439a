// csg_local.hip -- chunk-local sketch + top-k: one workgroup per chunk, the
// chunk's transpose built in LDS.
//
// The reference computes the similarity of row r from the global CSC: for
// each column c of r (CSR order), the rows of c in ascending order, kept only
// when they fall inside r's chunk (sporder/src/common/chunk_similarity_top_k.cu
// :53-83).  Restricted to one chunk, those rows are exactly the chunk's own
// rows holding c, so the global transpose (a device-wide sort of every
// nonzero) and the random CSC walks can be replaced by a transpose of the
// chunk's row block alone:
//
//   1. keys (c << lb) | local_row for the chunk's E nonzeros go to LDS;
//   2. a bitonic sort in LDS orders them by (column, row);
//   3. a row whose columns all occur once in the chunk has no candidates and
//      gets the all-zero table row at once;
//   4. other rows (one wave each) binary-search each column's run of keys in
//      LDS and feed the run's rows, ascending, to the wave64 sketch.
//
// The stream, and therefore the table, is identical to the reference's.
// Chunks with more nonzeros than kLocalKeyCap are appended to an overflow list
// for the global-CSC kernel.  Requires ceil(log2 n) + ceil(log2 C) <= 32 and
// C <= kLocalRowCap (checked by the host).
#include "common.hpp"
#include "sketch.hpp"

namespace sporder_hip {

namespace {

constexpr int kLocalThreads = 1024;
constexpr int kLocalWaves = kLocalThreads / kWave;

// First index in [0, count) with keys[i] > bound (keys sorted ascending).
__device__ __forceinline__ int32_t lds_upper_bound(const uint32_t *keys, int32_t count,
                                                   uint32_t bound) {
  int32_t lo = 0, hi = count;
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

// First index in [0, count) with keys[i] >= bound.
__device__ __forceinline__ int32_t lds_lower_bound(const uint32_t *keys, int32_t count,
                                                   uint32_t bound) {
  int32_t lo = 0, hi = count;
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

template <int CELLS>
__global__ void __launch_bounds__(kLocalThreads)
    chunk_local_sketch_kernel(int32_t n, int32_t k, int32_t chunk_size, int32_t lb,
                              const int32_t *__restrict__ row_ptr,
                              const int32_t *__restrict__ col_ind,
                              uint64_t *__restrict__ table, int32_t *__restrict__ overflow,
                              int32_t *__restrict__ overflow_count) {
  __shared__ uint32_t s_keys[kLocalKeyCap];
  __shared__ int32_t s_size[kLocalRowCap];
  __shared__ uint8_t s_multi[kLocalRowCap];

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;
  const int32_t chunk = blockIdx.x;
  const int32_t cs = chunk * chunk_size;
  const int32_t ce = (n - cs > chunk_size) ? cs + chunk_size : n;
  const int32_t rows = ce - cs;
  const int32_t e0 = row_ptr[cs];
  const int32_t E = row_ptr[ce] - e0;
  if (E > kLocalKeyCap) {
    if (tid == 0) overflow[atomicAdd(overflow_count, 1)] = chunk;
    return;
  }
  const uint32_t rmask = (lb == 0) ? 0u : ((1u << lb) - 1u);
  int32_t epad = 1;
  while (epad < E) epad <<= 1;

  // Stage the chunk's column indices with coalesced loads, then let one
  // thread per row turn its entries into (column << lb | local row) keys.
  for (int32_t i = tid; i < E; i += kLocalThreads) {
    s_keys[i] = static_cast<uint32_t>(col_ind[e0 + i]);
  }
  for (int32_t i = E + tid; i < epad; i += kLocalThreads) s_keys[i] = 0xFFFFFFFFu;
  for (int32_t r = tid; r < rows; r += kLocalThreads) {
    s_size[r] = row_ptr[cs + r + 1] - row_ptr[cs + r];
    s_multi[r] = 0;
  }
  __syncthreads();
  for (int32_t r = tid; r < rows; r += kLocalThreads) {
    const int32_t off = row_ptr[cs + r] - e0;
    const int32_t len = s_size[r];
    for (int32_t q = 0; q < len; ++q) {
      s_keys[off + q] = (s_keys[off + q] << lb) | static_cast<uint32_t>(r);
    }
  }
  __syncthreads();

  // Bitonic sort of s_keys[0, epad).
  for (int32_t kk = 2; kk <= epad; kk <<= 1) {
    for (int32_t j = kk >> 1; j > 0; j >>= 1) {
      for (int32_t i = tid; i < (epad >> 1); i += kLocalThreads) {
        const int32_t lo = ((i & ~(j - 1)) << 1) | (i & (j - 1));
        const int32_t hi = lo + j;
        const uint32_t a = s_keys[lo], b = s_keys[hi];
        const bool asc = (lo & kk) == 0;
        if (asc ? (a > b) : (a < b)) {
          s_keys[lo] = b;
          s_keys[hi] = a;
        }
      }
      __syncthreads();
    }
  }

  // Rows holding a column that another chunk row also holds.
  for (int32_t i = tid; i < E; i += kLocalThreads) {
    const uint32_t key = s_keys[i];
    const uint32_t c = key >> lb;
    const bool multi = (i > 0 && (s_keys[i - 1] >> lb) == c) ||
                       (i + 1 < E && (s_keys[i + 1] >> lb) == c);
    if (multi) s_multi[key & rmask] = 1;
  }
  __syncthreads();

  WaveSketch<CELLS> store;
  for (int32_t r = wave; r < rows; r += kLocalWaves) {
    const int32_t row = cs + r;
    uint64_t *out = table + static_cast<size_t>(row) * k;
    const int32_t row_size = s_size[r];
    if (row_size == 0 || s_multi[r] == 0) {
      for (int32_t j = lane; j < k; j += kWave) out[j] = 0;
      continue;
    }
    store.clear();
    const int32_t rb = row_ptr[row], re = rb + row_size;
    for (int32_t pb = rb; pb < re; pb += kWave) {
      const int32_t p = pb + lane;
      int32_t a = 0, b = 0;
      if (p < re) {
        const uint32_t base = static_cast<uint32_t>(col_ind[p]) << lb;
        a = lds_lower_bound(s_keys, E, base);
        b = lds_upper_bound(s_keys, E, base | rmask);
      }
      const int32_t len = b - a;
      const int32_t incl = wave_incl_scan(len);
      const int32_t excl = incl - len;
      const int32_t total = readlane(incl, kWave - 1);
      for (int32_t f0 = 0; f0 < total; f0 += kWave) {
        const int32_t f = f0 + lane;
        int32_t j = 0;
#pragma unroll
        for (int step = 32; step > 0; step >>= 1) {
          const int32_t t = j + step;
          const int32_t e = __shfl(excl, t & (kWave - 1), kWave);
          if (t < kWave && e <= f) j = t;
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
        uint64_t mask = ballot(item);
        while (mask) {
          const int i = __builtin_ctzll(mask);
          store.add(readlane(other, i), readlane_f(alpha, i));
          mask &= mask - 1;
        }
      }
    }
    store.select_top_k(k, out);
  }
}

template <int CELLS>
void launch_local(Context &ctx, int32_t n, int32_t k, int32_t chunk_size, int32_t lb,
                  const int32_t *d_ptr, const int32_t *d_ind, uint64_t *d_table,
                  int32_t *d_overflow, int32_t *d_overflow_count) {
  const int64_t chunks = ceil_div64(n, chunk_size);
  chunk_local_sketch_kernel<CELLS><<<dim3(static_cast<unsigned>(chunks)), kLocalThreads, 0,
                                     ctx.stream>>>(n, k, chunk_size, lb, d_ptr, d_ind, d_table,
                                                   d_overflow, d_overflow_count);
  SP_LAUNCH_CHECK();
}

} // namespace

bool chunk_local_supported(int32_t n, int32_t chunk_size) {
  return chunk_size <= kLocalRowCap && bits_for(n - 1) + bits_for(chunk_size - 1) <= 32;
}

void chunk_local_sketch_top_k(Context &ctx, int32_t n, int32_t k, int32_t chunk_size,
                              int32_t m_capacity, const int32_t *d_ptr, const int32_t *d_ind,
                              uint64_t *d_table, int32_t *d_overflow,
                              int32_t *d_overflow_count) {
  SP_EXPECT(k <= 256, "k must be <= 256");
  SP_EXPECT(chunk_local_supported(n, chunk_size), "chunk-local sketch not applicable");
  const int32_t lb = bits_for(chunk_size - 1);
  switch (m_capacity / 32) {
#define SP_CASE(C)                                                                       \
  case C:                                                                                \
    launch_local<C>(ctx, n, k, chunk_size, lb, d_ptr, d_ind, d_table, d_overflow,        \
                    d_overflow_count);                                                   \
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
