// scan.hip -- device-wide int32 prefix sums (exclusive or inclusive).
// Replaces the reference's cub::DeviceScan calls
// (sporder/src/common/csr2csc.cu:99-108, sporder/src/reorder.cu:87-98).
//
// Passes over 4096-element tiles: per-tile totals, then a per-tile scan with
// the tile's offset, which each workgroup sums from the totals before it when
// there are at most kDirectTiles tiles (16 MiB of input), and which one
// workgroup scanning the totals supplies otherwise.  Each tile is staged
// through LDS so HBM reads and writes stay coalesced.  A caller that already
// has the tile totals (a kernel that produced the input) starts at the
// second pass (scan_i32_from_totals).
#include "common.hpp"

namespace sporder_hip {

namespace {

constexpr int kScanBlock = 256;
constexpr int kScanItems = 16;
constexpr int kScanTile = kScanBlock * kScanItems;
static_assert(kScanTile == kScanTileElems, "scan tile size");
constexpr int64_t kDirectTiles = 4096;

// Block-wide exclusive scan of one value per thread; returns the block total
// through *total.
__device__ int32_t block_excl_scan(int32_t v, int32_t *total) {
  __shared__ int32_t wave_tot[kScanBlock / kWave];
  int tid = threadIdx.x;
  int lane = tid & (kWave - 1), wave = tid / kWave;
  int32_t incl = wave_incl_scan(v);
  if (lane == kWave - 1) wave_tot[wave] = incl;
  __syncthreads();
  int32_t before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kScanBlock / kWave; ++w) {
    int32_t t = wave_tot[w];
    before += (w < wave) ? t : 0;
    all += t;
  }
  __syncthreads();
  *total = all;
  return before + incl - v;
}

__global__ void __launch_bounds__(kScanBlock)
    scan_tile_totals(const int32_t *__restrict__ in, int64_t count,
                     int32_t *__restrict__ totals) {
  int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
  int32_t s = 0;
#pragma unroll
  for (int r = 0; r < kScanItems; ++r) {
    int64_t i = base + r * kScanBlock + threadIdx.x;
    if (i < count) s += in[i];
  }
  int32_t total;
  block_excl_scan(s, &total);
  if (threadIdx.x == 0) totals[blockIdx.x] = total;
}

// One workgroup: exclusive scan of the tile totals in place.
__global__ void __launch_bounds__(kScanBlock)
    scan_totals(int32_t *__restrict__ totals, int64_t num_tiles) {
  int32_t carry = 0;
  for (int64_t base = 0; base < num_tiles; base += kScanBlock) {
    int64_t i = base + threadIdx.x;
    int32_t v = i < num_tiles ? totals[i] : 0;
    int32_t total;
    int32_t ex = block_excl_scan(v, &total);
    if (i < num_tiles) totals[i] = carry + ex;
    carry += total;
  }
}

// `offsets` holds the tiles' exclusive offsets, or, with `direct`, their
// totals, which the workgroup sums up to its own tile.
__global__ void __launch_bounds__(kScanBlock)
    scan_tiles(const int32_t *in, int32_t *out, int64_t count,
               const int32_t *__restrict__ offsets, bool inclusive, bool direct) {
  __shared__ int32_t tile[kScanTile + kScanTile / 32];
  int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
  int tid = threadIdx.x;
  // The first totals (or the offset) are loaded before the tile, so their
  // latency overlaps the tile's loads.
  int32_t part = direct ? (tid < static_cast<int>(blockIdx.x) ? offsets[tid] : 0)
                        : (tid == 0 ? offsets[blockIdx.x] : 0);
  // Striped, coalesced load; padding of one word per 32 avoids bank
  // conflicts in the blocked pass below.
#pragma unroll
  for (int r = 0; r < kScanItems; ++r) {
    int e = r * kScanBlock + tid;
    int64_t i = base + e;
    tile[e + (e >> 5)] = i < count ? in[i] : 0;
  }
  if (direct) {
    for (int64_t t = tid + kScanBlock; t < blockIdx.x; t += kScanBlock) part += offsets[t];
  }
  int32_t offset;
  block_excl_scan(part, &offset);
  int32_t items[kScanItems];
  int32_t s = 0;
#pragma unroll
  for (int j = 0; j < kScanItems; ++j) {
    int e = tid * kScanItems + j;
    items[j] = tile[e + (e >> 5)];
    s += items[j];
  }
  int32_t total;
  int32_t run = block_excl_scan(s, &total) + offset;
#pragma unroll
  for (int j = 0; j < kScanItems; ++j) {
    int e = tid * kScanItems + j;
    int32_t v = items[j];
    tile[e + (e >> 5)] = inclusive ? run + v : run;
    run += v;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kScanItems; ++r) {
    int e = r * kScanBlock + tid;
    int64_t i = base + e;
    if (i < count) out[i] = tile[e + (e >> 5)];
  }
}

} // namespace

size_t scan_tmp_elems(int64_t count) {
  return static_cast<size_t>(ceil_div64(count, kScanTile) + 1);
}

void scan_i32_from_totals(Context &ctx, const int32_t *in, int32_t *out, int64_t count,
                          bool inclusive, int32_t *totals) {
  if (count <= 0) return;
  const int64_t tiles = ceil_div64(count, kScanTile);
  const bool direct = tiles <= kDirectTiles;
  if (!direct) {
    scan_totals<<<1, kScanBlock, 0, ctx.stream>>>(totals, tiles);
    SP_LAUNCH_CHECK();
  }
  scan_tiles<<<dim3(static_cast<unsigned>(tiles)), kScanBlock, 0, ctx.stream>>>(
      in, out, count, totals, inclusive, direct);
  SP_LAUNCH_CHECK();
}

void scan_i32(Context &ctx, const int32_t *in, int32_t *out, int64_t count,
              bool inclusive, int32_t *tmp) {
  if (count <= 0) return;
  int64_t tiles = ceil_div64(count, kScanTile);
  scan_tile_totals<<<dim3(static_cast<unsigned>(tiles)), kScanBlock, 0,
                     ctx.stream>>>(in, count, tmp);
  SP_LAUNCH_CHECK();
  scan_i32_from_totals(ctx, in, out, count, inclusive, tmp);
}

} // namespace sporder_hip
