// radix.hip -- stable LSD radix sort of (u32 key, u32 value) pairs, and the
// stable CSR -> CSC transpose built on it.
//
// Reference counterpart: sporder/src/common/csr2csc.cu:38-115 (copy keys,
// fill row ids, cub::DeviceRadixSort::SortPairs over 32 key bits, histogram +
// exclusive scan for col_ptr).  Here only the bits that can be set are sorted
// (ceil(log2 n) bits, 8 per pass), and col_ptr comes from the sorted keys
// without atomics.
//
// One pass = per-tile digit histograms -> one exclusive scan over the
// digit-major histogram table -> stable scatter.  Stability inside a tile
// comes from processing the tile in 256-item rounds in index order; within
// a round each wave ranks its 64 items by matching digits with 8 ballots.
#include "common.hpp"

namespace sporder_hip {

namespace {

constexpr int kRsBlock = 256;
constexpr int kRsWaves = kRsBlock / kWave;
constexpr int kRsRounds = 16;
constexpr int kRsTile = kRsBlock * kRsRounds;
constexpr int kRsDigits = 256;

__global__ void __launch_bounds__(kRsBlock)
    rs_histogram(const uint32_t *__restrict__ keys, int64_t count, int shift,
                 int32_t *__restrict__ hist, int64_t num_tiles) {
  __shared__ int32_t cnt[kRsDigits];
  int tid = threadIdx.x;
  cnt[tid] = 0;
  __syncthreads();
  int64_t base = static_cast<int64_t>(blockIdx.x) * kRsTile;
#pragma unroll 4
  for (int r = 0; r < kRsRounds; ++r) {
    int64_t i = base + r * kRsBlock + tid;
    if (i < count) atomicAdd(&cnt[(keys[i] >> shift) & 0xFF], 1);
  }
  __syncthreads();
  hist[static_cast<int64_t>(tid) * num_tiles + blockIdx.x] = cnt[tid];
}

__global__ void __launch_bounds__(kRsBlock)
    rs_scatter(const uint32_t *__restrict__ keys_in,
               const uint32_t *__restrict__ vals_in, int64_t count, int shift,
               const int32_t *__restrict__ offsets, int64_t num_tiles,
               uint32_t *__restrict__ keys_out,
               uint32_t *__restrict__ vals_out) {
  __shared__ int32_t digit_base[kRsDigits];
  __shared__ int32_t wave_cnt[kRsWaves][kRsDigits];
  int tid = threadIdx.x;
  int lane = tid & (kWave - 1), wave = tid / kWave;
  digit_base[tid] =
      offsets[static_cast<int64_t>(tid) * num_tiles + blockIdx.x];
  const uint64_t lanes_below = (uint64_t(1) << lane) - 1;
  int64_t base = static_cast<int64_t>(blockIdx.x) * kRsTile;

  for (int r = 0; r < kRsRounds; ++r) {
#pragma unroll
    for (int w = 0; w < kRsWaves; ++w) wave_cnt[w][tid] = 0;
    __syncthreads();

    int64_t i = base + r * kRsBlock + tid;
    bool valid = i < count;
    uint32_t key = valid ? keys_in[i] : 0u;
    uint32_t val = valid ? vals_in[i] : 0u;
    int d = static_cast<int>((key >> shift) & 0xFF);
    uint64_t peers = ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      bool bit = (d >> b) & 1;
      uint64_t m = ballot(bit);
      peers &= bit ? m : ~m;
    }
    int rank = __popcll(peers & lanes_below);
    if (valid && rank == 0) wave_cnt[wave][d] = __popcll(peers);
    __syncthreads();

    if (valid) {
      int32_t pos = digit_base[d] + rank;
      for (int w = 0; w < wave; ++w) pos += wave_cnt[w][d];
      keys_out[pos] = key;
      vals_out[pos] = val;
    }
    __syncthreads();
    int32_t add = 0;
#pragma unroll
    for (int w = 0; w < kRsWaves; ++w) add += wave_cnt[w][tid];
    digit_base[tid] += add;
    // The clear at the top of the next round follows a barrier-free window,
    // so fence it off from the reads above.
    __syncthreads();
  }
}

__global__ void copy_u32(const uint32_t *__restrict__ a, uint32_t *__restrict__ b,
                         int64_t count) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
       i < count; i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    b[i] = a[i];
  }
}

// row_ids[p] = row for every entry p of the row (one wave per row).
__global__ void fill_row_ids(int32_t n, const int32_t *__restrict__ ptr,
                             uint32_t *__restrict__ row_ids) {
  int lane = lane_id();
  int64_t wave = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) /
                 kWave;
  int64_t waves = static_cast<int64_t>(gridDim.x) * blockDim.x / kWave;
  for (int64_t row = wave; row < n; row += waves) {
    int32_t s = ptr[row], e = ptr[row + 1];
    for (int32_t p = s + lane; p < e; p += kWave) {
      row_ids[p] = static_cast<uint32_t>(row);
    }
  }
}

// col_ptr[c] = first position of a key >= c in the sorted key array.
__global__ void col_ptr_from_sorted(int32_t n, int32_t nnz,
                                    const uint32_t *__restrict__ sorted,
                                    int32_t *__restrict__ col_ptr) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
       i <= nnz; i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t cur = i < nnz ? static_cast<int64_t>(sorted[i]) : n;
    int64_t prev = i > 0 ? static_cast<int64_t>(sorted[i - 1]) : -1;
    for (int64_t c = prev + 1; c <= cur; ++c) {
      col_ptr[c] = static_cast<int32_t>(i);
    }
  }
}

} // namespace

size_t radix_tmp_elems(int64_t count) {
  int64_t tiles = ceil_div64(count, kRsTile);
  int64_t hist = tiles * kRsDigits;
  return static_cast<size_t>(hist + static_cast<int64_t>(scan_tmp_elems(hist)));
}

void radix_sort_pairs(Context &ctx, const uint32_t *keys_in,
                      const uint32_t *vals_in, uint32_t *keys_out,
                      uint32_t *vals_out, uint32_t *keys_alt,
                      uint32_t *vals_alt, int64_t count, int key_bits,
                      int32_t *tmp) {
  if (count <= 0) return;
  int passes = (key_bits + 7) / 8;
  if (passes == 0) {
    int g = ctx.grid_for(ceil_div64(count, 256), 256);
    copy_u32<<<g, 256, 0, ctx.stream>>>(keys_in, keys_out, count);
    SP_LAUNCH_CHECK();
    copy_u32<<<g, 256, 0, ctx.stream>>>(vals_in, vals_out, count);
    SP_LAUNCH_CHECK();
    return;
  }
  int64_t tiles = ceil_div64(count, kRsTile);
  int64_t hist_elems = tiles * kRsDigits;
  int32_t *hist = tmp;
  int32_t *scan_tmp = tmp + hist_elems;
  const uint32_t *ks = keys_in, *vs = vals_in;
  for (int pass = 0; pass < passes; ++pass) {
    // Land the last pass in *_out: alternate so that pass (passes-1) writes
    // the output buffers.
    bool to_out = ((passes - 1 - pass) % 2) == 0;
    uint32_t *kd = to_out ? keys_out : keys_alt;
    uint32_t *vd = to_out ? vals_out : vals_alt;
    int shift = pass * 8;
    rs_histogram<<<dim3(static_cast<unsigned>(tiles)), kRsBlock, 0,
                   ctx.stream>>>(ks, count, shift, hist, tiles);
    SP_LAUNCH_CHECK();
    scan_i32(ctx, hist, hist, hist_elems, false, scan_tmp);
    rs_scatter<<<dim3(static_cast<unsigned>(tiles)), kRsBlock, 0,
                 ctx.stream>>>(ks, vs, count, shift, hist, tiles, kd, vd);
    SP_LAUNCH_CHECK();
    ks = kd;
    vs = vd;
  }
}

size_t csr2csc_ws_bytes(int32_t n, int32_t nnz) {
  (void)n;
  size_t m = static_cast<size_t>(nnz);
  return 4 * ws_bytes<uint32_t>(m) + ws_bytes<int32_t>(radix_tmp_elems(nnz));
}

void csr2csc(Context &ctx, int32_t n, int32_t nnz, const int32_t *d_ptr,
             const int32_t *d_ind, int32_t *d_col_ptr, int32_t *d_row_ind) {
  uint32_t *row_ids = ctx.take<uint32_t>(nnz);
  uint32_t *keys_sorted = ctx.take<uint32_t>(nnz);
  uint32_t *keys_alt = ctx.take<uint32_t>(nnz);
  uint32_t *vals_alt = ctx.take<uint32_t>(nnz);
  int32_t *tmp = ctx.take<int32_t>(radix_tmp_elems(nnz));
  if (nnz > 0) {
    int g = ctx.grid_for(ceil_div64(n, 4), 256);
    fill_row_ids<<<g, 256, 0, ctx.stream>>>(n, d_ptr, row_ids);
    SP_LAUNCH_CHECK();
    radix_sort_pairs(ctx, reinterpret_cast<const uint32_t *>(d_ind), row_ids,
                     keys_sorted, reinterpret_cast<uint32_t *>(d_row_ind),
                     keys_alt, vals_alt, nnz, bits_for(n - 1), tmp);
  }
  int g = ctx.grid_for(ceil_div64(static_cast<int64_t>(nnz) + 1, 256), 256);
  col_ptr_from_sorted<<<g, 256, 0, ctx.stream>>>(n, nnz, keys_sorted, d_col_ptr);
  SP_LAUNCH_CHECK();
}

} // namespace sporder_hip
