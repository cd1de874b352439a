// pillars.hip -- sporder_count_pillars: distinct columns per window of
// `height` consecutive rows, summed over the windows.
//
// Reference: sporder/src/count_pillars.cu:11-85 (keys (window << 32 | column)
// of every nonzero, a device radix sort, then a count of key changes) and the
// bridge sporder/src/sporder.cpp:62-67.  Here a window's nonzeros are one
// contiguous CSR range, so most windows are handled where they lie:
//   - one wave per window copies the window's columns to its LDS slice
//     (kWinCap entries), sorts them there (bitonic, wave_sort.hpp) and counts
//     the positions where the value changes;
//   - windows with more nonzeros are listed; their columns are gathered into
//     one array and sorted by column and then, stably, by window, and the
//     (window, column) changes are counted.
// Columns need not be sorted or distinct within a row (duplicates count once),
// as the reference documents.
#include "common.hpp"
#include "wave_sort.hpp"

#include <algorithm>

namespace sporder_hip {

namespace {

constexpr int kWinCap = 4096;
constexpr int kPillarBlock = 256;
constexpr int kPillarWaves = kPillarBlock / kWave;

__global__ void __launch_bounds__(kPillarBlock)
    pillar_windows(int32_t n, int32_t height, const int32_t *__restrict__ ptr,
                   const int32_t *__restrict__ ind, unsigned long long *total,
                   int32_t *__restrict__ big, int32_t *__restrict__ big_count) {
  __shared__ uint32_t s_cols[kPillarWaves][kWinCap];
  const int lane = lane_id();
  uint32_t *a = s_cols[threadIdx.x / kWave];
  const int64_t windows = ceil_div64(n, height);
  const int64_t wave0 = static_cast<int64_t>(blockIdx.x) * kPillarWaves + threadIdx.x / kWave;
  const int64_t nwaves = static_cast<int64_t>(gridDim.x) * kPillarWaves;
  unsigned long long mine = 0;
  for (int64_t w = wave0; w < windows; w += nwaves) {
    const int64_t r0 = w * height;
    const int64_t r1 = r0 + height < n ? r0 + height : n;
    const int32_t s = ptr[r0], e = ptr[r1];
    const int32_t len = e - s;
    if (len > kWinCap) {
      if (lane == 0) big[atomicAdd(big_count, 1)] = static_cast<int32_t>(w);
      continue;
    }
    for (int32_t i = lane; i < len; i += kWave) a[i] = static_cast<uint32_t>(ind[s + i]);
    wave_lds_fence();
    wave_sort_lds(a, len);
    uint32_t changes = 0;
    for (int32_t i = lane; i < len; i += kWave) changes += (i == 0 || a[i] != a[i - 1]);
    mine += static_cast<uint32_t>(wave_sum(static_cast<int32_t>(changes)));
    wave_lds_fence(); // the next window overwrites the slice
  }
  if (lane == 0 && mine) atomicAdd(total, mine);
}

__global__ void big_lengths(int32_t n, int32_t height, const int32_t *__restrict__ ptr,
                            const int32_t *__restrict__ big, int32_t bcount,
                            int32_t *__restrict__ len) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i <= bcount;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    if (i < bcount) {
      const int64_t r0 = static_cast<int64_t>(big[i]) * height;
      const int64_t r1 = r0 + height < n ? r0 + height : n;
      len[i] = ptr[r1] - ptr[r0];
    } else {
      len[i] = 0;
    }
  }
}

// One workgroup per listed window: its columns and its rank.
__global__ void big_gather(int32_t n, int32_t height, const int32_t *__restrict__ ptr,
                           const int32_t *__restrict__ ind, const int32_t *__restrict__ big,
                           int32_t bcount, const int32_t *__restrict__ off,
                           uint32_t *__restrict__ cols, uint32_t *__restrict__ rank) {
  for (int32_t i = blockIdx.x; i < bcount; i += gridDim.x) {
    const int32_t s = ptr[static_cast<int64_t>(big[i]) * height];
    const int32_t g0 = off[i], len = off[i + 1] - g0;
    for (int32_t t = threadIdx.x; t < len; t += blockDim.x) {
      cols[g0 + t] = static_cast<uint32_t>(ind[s + t]);
      rank[g0 + t] = static_cast<uint32_t>(i);
    }
  }
}

// Sorted by (rank, column): count the positions where either changes.
__global__ void count_changes(int64_t count, const uint32_t *__restrict__ rank,
                              const uint32_t *__restrict__ cols,
                              unsigned long long *total) {
  uint32_t mine = 0;
  for (int64_t q = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; q < count;
       q += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    mine += (q == 0 || rank[q] != rank[q - 1] || cols[q] != cols[q - 1]);
  }
  const int32_t s = wave_sum(static_cast<int32_t>(mine));
  if (lane_id() == 0 && s) atomicAdd(total, static_cast<unsigned long long>(s));
}

__global__ void gather_u32(int64_t count, const uint32_t *__restrict__ src,
                           const uint32_t *__restrict__ idx, uint32_t *__restrict__ dst) {
  for (int64_t q = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; q < count;
       q += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    dst[q] = src[idx[q]];
  }
}

__global__ void iota_u32(int64_t count, uint32_t *__restrict__ dst) {
  for (int64_t q = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; q < count;
       q += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    dst[q] = static_cast<uint32_t>(q);
  }
}

} // namespace

} // namespace sporder_hip

using namespace sporder_hip;

extern "C" void sporder_count_pillars(sporder_context_t h, int32_t n, int32_t nnz,
                                      const int32_t *d_ptr, const int32_t *d_ind,
                                      int32_t height, int32_t *count) {
  SP_EXPECT(h != nullptr, "null context");
  SP_EXPECT(height >= 1, "height must be >= 1");
  SP_EXPECT(n >= 1 && nnz >= 0, "expect n >= 1 and nnz >= 0");
  SP_EXPECT(count != nullptr, "count must not be null");
  Context &ctx = h->impl;
  if (nnz == 0) {
    *count = 0;
    return;
  }
  const int64_t windows = ceil_div64(n, height);
  ctx.reserve(ws_bytes<unsigned long long>(1) + ws_bytes<int32_t>(2) +
              ws_bytes<int32_t>(static_cast<size_t>(windows)) +
              ws_bytes<int32_t>(static_cast<size_t>(windows) + 1) +
              ws_bytes<int32_t>(scan_tmp_elems(windows + 1)));
  auto *total = ctx.take<unsigned long long>(1);
  int32_t *big_count = ctx.take<int32_t>(2);
  int32_t *big = ctx.take<int32_t>(static_cast<size_t>(windows));
  int32_t *off = ctx.take<int32_t>(static_cast<size_t>(windows) + 1);
  int32_t *scan_tmp = ctx.take<int32_t>(scan_tmp_elems(windows + 1));
  fill_u32(ctx, total, 2, 0u);
  fill_u32(ctx, big_count, 1, 0u);
  const int g = ctx.grid_for(ceil_div64(windows, kPillarWaves), kPillarBlock, 2);
  pillar_windows<<<g, kPillarBlock, 0, ctx.stream>>>(n, height, d_ptr, d_ind, total, big,
                                                      big_count);
  SP_LAUNCH_CHECK();
  int32_t bcount = 0;
  SP_HIP(hipMemcpyAsync(&bcount, big_count, sizeof(int32_t), hipMemcpyDeviceToHost,
                        ctx.stream));
  ctx.sync();
  if (bcount > 0) {
    const int g1 = ctx.grid_for(ceil_div64(static_cast<int64_t>(bcount) + 1, 256), 256, 4);
    big_lengths<<<g1, 256, 0, ctx.stream>>>(n, height, d_ptr, big, bcount, off);
    SP_LAUNCH_CHECK();
    scan_i32(ctx, off, off, static_cast<int64_t>(bcount) + 1, false, scan_tmp);
    int32_t H32 = 0;
    SP_HIP(hipMemcpyAsync(&H32, off + bcount, sizeof(int32_t), hipMemcpyDeviceToHost,
                          ctx.stream));
    ctx.sync();
    const size_t H = static_cast<size_t>(H32);
    const size_t tmp_elems = radix_tmp_elems(H32);
    auto *base = static_cast<uint32_t *>(ctx.aux_reserve((8 * H + tmp_elems) * 4 + 10 * 256));
    auto carve = [&](size_t elems) {
      uint32_t *p = base;
      base += (elems + 63) & ~size_t(63);
      return p;
    };
    uint32_t *cols = carve(H), *rank = carve(H), *idx = carve(H), *c1 = carve(H);
    uint32_t *v1 = carve(H), *ka = carve(H), *va = carve(H), *r2 = carve(H);
    int32_t *tmp = reinterpret_cast<int32_t *>(carve(tmp_elems));
    big_gather<<<std::min<int32_t>(bcount, ctx.num_cus * 8), 256, 0, ctx.stream>>>(
        n, height, d_ptr, d_ind, big, bcount, off, cols, rank);
    SP_LAUNCH_CHECK();
    const int gq = ctx.grid_for(ceil_div64(H32, 256), 256, 4);
    iota_u32<<<gq, 256, 0, ctx.stream>>>(H32, idx);
    SP_LAUNCH_CHECK();
    // Stable by column, then stable by window rank: (rank, column) order.
    radix_sort_pairs(ctx, cols, idx, c1, v1, ka, va, H32, bits_for(n - 1), tmp);
    gather_u32<<<gq, 256, 0, ctx.stream>>>(H32, rank, v1, r2);
    SP_LAUNCH_CHECK();
    radix_sort_pairs(ctx, r2, c1, rank, cols, ka, va, H32, bits_for(bcount - 1), tmp);
    count_changes<<<gq, 256, 0, ctx.stream>>>(H32, rank, cols, total);
    SP_LAUNCH_CHECK();
  }
  unsigned long long host_total = 0;
  SP_HIP(hipMemcpyAsync(&host_total, total, sizeof(host_total), hipMemcpyDeviceToHost,
                        ctx.stream));
  ctx.sync();
  *count = static_cast<int32_t>(host_total);
}
