// spmm_plan.hip -- SpMM plans: blocks of rows that share each B-row load.
//
// The reference's SpMM harness converts each matrix once, untimed, in
// SpMMMethod.prepare (bench/spmm/spmm_bench/base.py:41-46), then times one
// launch per run() (base.py:48-59); the C hook times cuSPARSE CSR ALG1
// (sporder/src/bench_cusparse_spmm.cu:51-100).  A plan is this library's
// prepare step for its CSR SpMM.
//
// Row blocks.  Rows are grouped in blocks of kBlockRows (8) consecutive rows.
// A block's entries are the distinct columns of its rows, ascending, each
// with the mask of the block rows that hold it.  One wave computes a block:
// per entry it loads the B row once and applies it to every row whose mask
// bit is set.  Entries are visited in ascending column order, so each row
// still sees its own nonzeros in CSR order: every C element is the same fmaf
// chain from 0.0f as the row-split's, bit for bit.  A band of half-width 8
// has 17 nonzeros per row but 3 entries per row (24 per block of 8), so the
// B rows a wave loads drop from 17 to 3 per row.
//
// Inspector (spmm_plan_tiles, one workgroup per tile of kSpmmTileRows rows,
// run twice: count, then write): each block's (column, row) keys are sorted
// in LDS; runs of equal columns are entries.  A tile is blocked when its
// entries are at most half its nonzeros, no row has more than
// SPORDER_SPMM_LONG_ROW nonzeros (those keep their segment launches) and no
// row holds a column twice; other tiles run the row-split over a tile list.
//
// Kernel (spmm_block_kernel, one wave per block): the lanes hold 64 entries
// at a time; each lane gathers the CSR values of its own entry (for row j,
// the value's rank among the row's entries comes from a ballot popcount), so
// a set mask bit costs one readlane plus VEC FMAs; the entry's mask selects a
// straight-line case per nibble of rows (a scalar switch), so no FMA is
// computed for a row that lacks the column.
#include "common.hpp"

#include <algorithm>
#include <vector>

namespace sporder_hip {
namespace {

constexpr int kPlanBlock = 256;
constexpr int kBlockRows = 8;
constexpr int kTileBlocks = kSpmmTileRows / kBlockRows;
constexpr int kPlanKeys = 4096; // keys of one block the inspector sorts
constexpr int kLongRowPlan = SPORDER_SPMM_LONG_ROW;
// B rows in flight per wave: 8, or 4 at 4 columns per lane (registers).
template <int VEC> constexpr int block_loads() { return VEC >= 4 ? 4 : 8; }

// Ascending bitonic sort of keys[0, m2) in LDS, m2 a power of two; every
// thread of the block calls it.
__device__ void block_bitonic(uint64_t *keys, int m2) {
  for (int k = 2; k <= m2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < m2; i += kPlanBlock) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const uint64_t a = keys[i], b = keys[ixj];
          const bool up = (i & k) == 0;
          if ((a > b) == up) {
            keys[i] = b;
            keys[ixj] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Count pass (write == false): ecount[tile * 8 + b] = entries of block b when
// the tile is blocked, 0 otherwise; kind[tile] = 1 when blocked.  Write pass:
// the entries (column, row mask) of each blocked tile's blocks at boff[block].
// Each block's (column << 3 | row) keys are sorted in LDS (a block holds at
// most 8 rows of at most SPORDER_SPMM_LONG_ROW nonzeros); a run of equal
// columns is one entry.  A tile in which a row holds a column twice is not
// blocked (one mask bit cannot stand for two values).
__global__ void __launch_bounds__(kPlanBlock)
    spmm_plan_tiles(int32_t n, const int32_t *__restrict__ ptr, const int32_t *__restrict__ ind,
                    bool write, int32_t *__restrict__ kind, int32_t *__restrict__ ecount,
                    const int32_t *__restrict__ boff, int2 *__restrict__ entries) {
  __shared__ uint64_t keys[kPlanKeys];
  __shared__ int32_t s_ptr[kSpmmTileRows + 1];
  __shared__ int32_t s_cnt[kTileBlocks];
  __shared__ int32_t s_scan[kPlanBlock / kWave];
  __shared__ int32_t s_long;
  __shared__ int32_t s_dup; // some row repeats a column inside the tile
  static_assert(kBlockRows * kLongRowPlan <= kPlanKeys, "a block's keys fit the sort");
  const int64_t tile = blockIdx.x;
  if (write && kind[tile] == 0) return;
  const int32_t r0 = static_cast<int32_t>(tile * kSpmmTileRows);
  const int32_t r1 = min(r0 + kSpmmTileRows, n);
  const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
  if (tid <= r1 - r0) s_ptr[tid] = ptr[r0 + tid];
  if (tid < kTileBlocks) s_cnt[tid] = 0;
  if (tid == 0) {
    s_long = 0;
    s_dup = 0;
  }
  __syncthreads();
  if (tid < r1 - r0 && s_ptr[tid + 1] - s_ptr[tid] > kLongRowPlan) atomicOr(&s_long, 1);
  __syncthreads();
  const int32_t m = s_ptr[r1 - r0] - s_ptr[0];
  if (s_long != 0 || m == 0) {
    if (!write && tid == 0) kind[tile] = 0;
    if (!write && tid < kTileBlocks) ecount[tile * kTileBlocks + tid] = 0;
    return;
  }
  for (int blk = 0; blk < kTileBlocks; ++blk) {
    const int32_t br0 = min(blk * kBlockRows, r1 - r0), br1 = min(br0 + kBlockRows, r1 - r0);
    const int32_t bp0 = s_ptr[br0], mb = s_ptr[br1] - bp0;
    if (mb == 0) continue; // uniform
    int m2 = kWave;
    while (m2 < mb) m2 <<= 1;
    for (int i = tid; i < m2; i += kPlanBlock) {
      uint64_t key = ~0ull;
      if (i < mb) {
        int j = 0; // the block row holding nonzero bp0 + i
        while (br0 + j + 1 < br1 && s_ptr[br0 + j + 1] - bp0 <= i) ++j;
        key = (static_cast<uint64_t>(ind[bp0 + i]) << 3) | static_cast<uint64_t>(j);
      }
      keys[i] = key;
    }
    __syncthreads();
    block_bitonic(keys, m2);
    // Entry starts (first key of each column), ranked by a block scan over
    // the runs of `per` sorted keys each thread owns.
    const int per = (m2 + kPlanBlock - 1) / kPlanBlock;
    const int a = tid * per, b = min(a + per, mb);
    int32_t cnt = 0;
    bool dup = false;
    for (int i = a; i < b; ++i) {
      cnt += i == 0 || (keys[i] >> 3) != (keys[i - 1] >> 3);
      // Equal (column, row) keys: a row that holds one column twice.  Its
      // entry would carry one mask bit for two values, so the tile stays on
      // the row-split, which adds both.
      dup = dup || (i > 0 && keys[i] == keys[i - 1]);
    }
    if (!write && dup) atomicOr(&s_dup, 1);
    const int32_t incl = wave_incl_scan(cnt);
    if (lane == kWave - 1) s_scan[wave] = incl;
    __syncthreads();
    int32_t o = incl - cnt, total = 0;
    for (int w = 0; w < kPlanBlock / kWave; ++w) {
      o += w < wave ? s_scan[w] : 0;
      total += s_scan[w];
    }
    if (write) {
      const int32_t base = boff[tile * kTileBlocks + blk];
      for (int i = a; i < b; ++i) {
        if (i == 0 || (keys[i] >> 3) != (keys[i - 1] >> 3)) {
          int32_t mask = 0;
          for (int t = i; t < mb && (keys[t] >> 3) == (keys[i] >> 3); ++t) {
            mask |= 1 << static_cast<int>(keys[t] & 7);
          }
          entries[base + o] = make_int2(static_cast<int32_t>(keys[i] >> 3), mask);
          ++o;
        }
      }
    } else if (tid == 0) {
      s_cnt[blk] = total;
    }
    __syncthreads(); // keys and s_scan are reused by the next block
  }
  if (!write) {
    const int32_t total = (s_cnt[0] + s_cnt[1] + s_cnt[2] + s_cnt[3]) +
                          (s_cnt[4] + s_cnt[5] + s_cnt[6] + s_cnt[7]);
    const bool blocked =
        s_dup == 0 && 2 * static_cast<int64_t>(total) <= static_cast<int64_t>(m);
    if (tid < kTileBlocks) ecount[tile * kTileBlocks + tid] = blocked ? s_cnt[tid] : 0;
    if (tid == 0) kind[tile] = blocked ? 1 : 0;
  }
}

template <int VEC> struct VecOf {
  typedef float T __attribute__((ext_vector_type(VEC)));
};

__device__ __forceinline__ float readlane_float(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// a + v * b per component, each a separate fmaf.
template <int VEC, typename V> __device__ __forceinline__ V vec_fma(float v, const V &b, V a) {
  a.x = fmaf(v, b.x, a.x);
  if constexpr (VEC >= 2) a.y = fmaf(v, b.y, a.y);
  if constexpr (VEC >= 4) {
    a.z = fmaf(v, b.z, a.z);
    a.w = fmaf(v, b.w, a.w);
  }
  return a;
}

// The FMAs of one entry for the rows of nibble J0 / 4 set in MASK: row j's
// value is w[j] in the entry's lane e.
template <int J0, int MASK, int VEC, typename V>
__device__ __forceinline__ void apply_rows(const V &bv, int e, const float (&w)[kBlockRows],
                                           V (&acc)[kBlockRows]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if ((MASK >> j) & 1) {
      acc[J0 + j] = vec_fma<VEC>(readlane_float(w[J0 + j], e), bv, acc[J0 + j]);
    }
  }
}

template <int J0, int VEC, typename V>
__device__ __forceinline__ void apply_nibble(int m4, const V &bv, int e,
                                             const float (&w)[kBlockRows], V (&acc)[kBlockRows]) {
  switch (m4) {
  case 0: break;
  case 1: apply_rows<J0, 1, VEC>(bv, e, w, acc); break;
  case 2: apply_rows<J0, 2, VEC>(bv, e, w, acc); break;
  case 3: apply_rows<J0, 3, VEC>(bv, e, w, acc); break;
  case 4: apply_rows<J0, 4, VEC>(bv, e, w, acc); break;
  case 5: apply_rows<J0, 5, VEC>(bv, e, w, acc); break;
  case 6: apply_rows<J0, 6, VEC>(bv, e, w, acc); break;
  case 7: apply_rows<J0, 7, VEC>(bv, e, w, acc); break;
  case 8: apply_rows<J0, 8, VEC>(bv, e, w, acc); break;
  case 9: apply_rows<J0, 9, VEC>(bv, e, w, acc); break;
  case 10: apply_rows<J0, 10, VEC>(bv, e, w, acc); break;
  case 11: apply_rows<J0, 11, VEC>(bv, e, w, acc); break;
  case 12: apply_rows<J0, 12, VEC>(bv, e, w, acc); break;
  case 13: apply_rows<J0, 13, VEC>(bv, e, w, acc); break;
  case 14: apply_rows<J0, 14, VEC>(bv, e, w, acc); break;
  default: apply_rows<J0, 15, VEC>(bv, e, w, acc); break;
  }
}

// One wave per block of kBlockRows rows of a blocked tile and slice of
// W = 64 * VEC columns of B and C (slices are separate workgroups, so no
// registers live across them).  Workgroups are mapped to tiles by
// xcd_block(), so each XCD takes a contiguous run of the tile list, whose
// neighbouring tiles share B rows in its L2.
template <int VEC>
__global__ void __launch_bounds__(kPlanBlock)
    spmm_block_kernel(int32_t n, const int32_t *__restrict__ tiles, int32_t ntiles,
                      const int32_t *__restrict__ ptr, const float *__restrict__ val,
                      const int2 *__restrict__ entries, const int32_t *__restrict__ boff,
                      int32_t N, const float *__restrict__ B, float *__restrict__ C) {
  typedef typename VecOf<VEC>::T V;
  constexpr int W = kWave * VEC;
  constexpr int kWaves = kPlanBlock / kWave;
  constexpr int kGroupsPerTile = kTileBlocks / kWaves;
  constexpr int U = block_loads<VEC>();
  const int gg = static_cast<int>(xcd_block());
  const int per_slice = ntiles * kGroupsPerTile;
  const int32_t cb = (gg / per_slice) * W;
  const int g = gg % per_slice;
  const int ti = g / kGroupsPerTile;
  if (ti >= ntiles || cb >= N) return;
  const int32_t blk = tiles[ti] * kTileBlocks + (g % kGroupsPerTile) * kWaves +
                      static_cast<int32_t>(threadIdx.x) / kWave;
  const int32_t r0 = blk * kBlockRows;
  if (r0 >= n) return;
  const int lane = lane_id();
  const int32_t nr = min(kBlockRows, n - r0);
  const int32_t pv = ptr[r0 + min(lane, nr)];
  const int32_t ev = boff[blk + min(lane, 1)];
  const int32_t E0 = readlane(ev, 0), E1 = readlane(ev, 1);
  int32_t rs[kBlockRows];
#pragma unroll
  for (int j = 0; j < kBlockRows; ++j) rs[j] = readlane(pv, min(j, nr));
  const uint64_t below = (1ull << lane) - 1ull;
  {
    V acc[kBlockRows];
    int32_t done[kBlockRows];
#pragma unroll
    for (int j = 0; j < kBlockRows; ++j) {
      acc[j] = static_cast<V>(0.0f);
      done[j] = 0;
    }
    for (int32_t eb = E0; eb < E1; eb += kWave) {
      const int32_t mc = min(kWave, E1 - eb);
      const int2 my = entries[min(eb + lane, E1 - 1)];
      const int32_t mymask = lane < mc ? my.y : 0;
      // w[j]: the value of (this lane's entry, row j): the row's nonzeros in
      // CSR order, ranked by the entries that hold row j.
      float w[kBlockRows];
#pragma unroll
      for (int j = 0; j < kBlockRows; ++j) {
        const bool bit = (mymask >> j) & 1;
        const uint64_t bal = ballot(bit);
        w[j] = bit ? val[rs[j] + done[j] + __popcll(bal & below)] : 0.0f;
        done[j] += __popcll(bal);
      }
      for (int32_t k = 0; k < mc; k += U) {
        V bv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int32_t c = readlane(my.x, min(k + u, kWave - 1));
          bv[u] = *reinterpret_cast<const V *>(B + static_cast<int64_t>(c) * N + cb + lane * VEC);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int e = min(k + u, kWave - 1);
          const int32_t mm = k + u < mc ? readlane(mymask, e) : 0;
          apply_nibble<0, VEC>(mm & 15, bv[u], e, w, acc);
          apply_nibble<4, VEC>((mm >> 4) & 15, bv[u], e, w, acc);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < kBlockRows; ++j) {
      if (j < nr) {
        __builtin_nontemporal_store(
            acc[j], reinterpret_cast<V *>(C + static_cast<int64_t>(r0 + j) * N + cb + lane * VEC));
      }
    }
  }
}

} // namespace
} // namespace sporder_hip

struct sporder_spmm_plan_struct {
  int device = 0;
  int32_t n = 0, nnz = 0;
  int2 *entries = nullptr;    // (column, row mask) per entry of the blocked tiles' blocks
  int32_t *boff = nullptr;    // each block's first entry (blocks + 1)
  int32_t *blocked = nullptr; // blocked tiles
  int32_t *direct = nullptr;  // the other tiles
  int32_t n_blocked = 0, n_direct = 0;
  bool long_rows = true; // some row passes SPORDER_SPMM_LONG_ROW nonzeros
  sporder_spmm_plan_info_t info{};
};

using namespace sporder_hip;

namespace {

template <typename T> T *dev_alloc(size_t count) {
  void *p = nullptr;
  SP_HIP(hipMalloc(&p, std::max<size_t>(count, 1) * sizeof(T)));
  return static_cast<T *>(p);
}

template <int VEC>
void launch_blocks(Context &ctx, const sporder_spmm_plan_struct &pl, const int32_t *ptr,
                   const float *val, int32_t N, const float *B, float *C) {
  const int64_t slices = N / (kWave * VEC);
  const int64_t grid =
      slices * static_cast<int64_t>(pl.n_blocked) * (kTileBlocks / (kPlanBlock / kWave));
  spmm_block_kernel<VEC><<<dim3(static_cast<unsigned>(grid)), kPlanBlock, 0, ctx.stream>>>(
      pl.n, pl.blocked, pl.n_blocked, ptr, val, pl.entries, pl.boff, N, B, C);
  SP_LAUNCH_CHECK();
}

} // namespace

extern "C" {

sporder_spmm_plan_t sporder_spmm_plan_create(sporder_context_t h, int32_t n, int32_t nnz,
                                             const int32_t *d_ptr, const int32_t *d_ind,
                                             sporder_spmm_plan_info_t *info) {
  SP_EXPECT(h != nullptr, "null context");
  SP_EXPECT(n >= 1 && nnz >= 0, "expect n >= 1 and nnz >= 0");
  Context &ctx = h->impl;
  auto *pl = new sporder_spmm_plan_struct;
  pl->device = ctx.device;
  pl->n = n;
  pl->nnz = nnz;
  const int64_t tiles = ceil_div64(n, kSpmmTileRows);
  const int64_t blocks = tiles * kTileBlocks;
  int32_t *kind = dev_alloc<int32_t>(static_cast<size_t>(tiles));
  int32_t *ecount = dev_alloc<int32_t>(static_cast<size_t>(blocks));
  pl->boff = dev_alloc<int32_t>(static_cast<size_t>(blocks) + 1);
  spmm_plan_tiles<<<dim3(static_cast<unsigned>(tiles)), kPlanBlock, 0, ctx.stream>>>(
      n, d_ptr, d_ind, false, kind, ecount, nullptr, nullptr);
  SP_LAUNCH_CHECK();
  std::vector<int32_t> hk(static_cast<size_t>(tiles)), hc(static_cast<size_t>(blocks)),
      hp(static_cast<size_t>(n) + 1);
  SP_HIP(hipMemcpyAsync(hk.data(), kind, hk.size() * 4, hipMemcpyDeviceToHost, ctx.stream));
  SP_HIP(hipMemcpyAsync(hc.data(), ecount, hc.size() * 4, hipMemcpyDeviceToHost, ctx.stream));
  SP_HIP(hipMemcpyAsync(hp.data(), d_ptr, hp.size() * 4, hipMemcpyDeviceToHost, ctx.stream));
  ctx.sync();
  std::vector<int32_t> off(static_cast<size_t>(blocks) + 1, 0), blocked, direct;
  for (int64_t b = 0; b < blocks; ++b) off[b + 1] = off[b] + hc[b];
  sporder_spmm_plan_info_t in{};
  in.tiles = static_cast<int32_t>(tiles);
  for (int64_t t = 0; t < tiles; ++t) {
    const int32_t r0 = static_cast<int32_t>(t * kSpmmTileRows);
    const int32_t r1 = std::min<int32_t>(r0 + kSpmmTileRows, n);
    if (hk[t] == 0) {
      direct.push_back(static_cast<int32_t>(t));
      continue;
    }
    blocked.push_back(static_cast<int32_t>(t));
    in.blocked_rows += r1 - r0;
    in.blocked_nnz += hp[r1] - hp[r0];
  }
  in.blocked_tiles = static_cast<int32_t>(blocked.size());
  pl->long_rows = false;
  for (int32_t r = 0; r < n && !pl->long_rows; ++r) pl->long_rows = hp[r + 1] - hp[r] > kLongRowPlan;
  in.entries = off[blocks];
  pl->entries = dev_alloc<int2>(static_cast<size_t>(off[blocks]));
  SP_HIP(hipMemcpyAsync(pl->boff, off.data(), off.size() * 4, hipMemcpyHostToDevice, ctx.stream));
  if (in.entries > 0) {
    spmm_plan_tiles<<<dim3(static_cast<unsigned>(tiles)), kPlanBlock, 0, ctx.stream>>>(
        n, d_ptr, d_ind, true, kind, ecount, pl->boff, pl->entries);
    SP_LAUNCH_CHECK();
  }
  pl->n_blocked = static_cast<int32_t>(blocked.size());
  pl->n_direct = static_cast<int32_t>(direct.size());
  pl->blocked = dev_alloc<int32_t>(blocked.size());
  pl->direct = dev_alloc<int32_t>(direct.size());
  if (!blocked.empty()) {
    SP_HIP(hipMemcpyAsync(pl->blocked, blocked.data(), blocked.size() * 4, hipMemcpyHostToDevice,
                          ctx.stream));
  }
  if (!direct.empty()) {
    SP_HIP(hipMemcpyAsync(pl->direct, direct.data(), direct.size() * 4, hipMemcpyHostToDevice,
                          ctx.stream));
  }
  ctx.sync();
  SP_HIP(hipFree(kind));
  SP_HIP(hipFree(ecount));
  pl->info = in;
  if (info) *info = in;
  return pl;
}

void sporder_spmm_plan_destroy(sporder_spmm_plan_t plan) {
  if (plan == nullptr) return;
  int cur = 0;
  SP_HIP(hipGetDevice(&cur));
  SP_HIP(hipSetDevice(plan->device));
  SP_HIP(hipFree(plan->entries));
  SP_HIP(hipFree(plan->boff));
  SP_HIP(hipFree(plan->blocked));
  SP_HIP(hipFree(plan->direct));
  SP_HIP(hipSetDevice(cur));
  delete plan;
}

void sporder_spmm_csr_plan(sporder_context_t h, sporder_spmm_plan_t plan, int32_t n,
                           int32_t nnz, const int32_t *d_ptr, const int32_t *d_ind,
                           const float *d_val, int32_t cols, const float *d_b, float *d_c,
                           float *kernel_ms) {
  SP_EXPECT(h != nullptr && plan != nullptr, "null context or plan");
  SP_EXPECT(plan->n == n && plan->nnz == nnz, "plan was made for another matrix size");
  SP_EXPECT(cols >= 1, "cols must be >= 1");
  Context &ctx = h->impl;
  SP_EXPECT(plan->device == ctx.device, "plan and context are on different devices");
  EventSpan t;
  t.create(kernel_ms != nullptr);
  const bool aligned = (reinterpret_cast<uintptr_t>(d_b) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(d_c) % 16 == 0);
  // Columns per lane: 4 when cols is a multiple of 256, 2 of 128, 1 of 64.
  const int vec = cols % 256 == 0 ? 4 : (cols % 128 == 0 ? 2 : (cols % 64 == 0 ? 1 : 0));
  t.begin(ctx.stream);
  if (!aligned || vec == 0 || plan->n_blocked == 0) {
    spmm_rowsplit_tiles(ctx, n, nnz, d_ptr, d_ind, d_val, cols, d_b, d_c, nullptr, 0,
                        plan->long_rows);
  } else {
    if (vec == 4) {
      launch_blocks<4>(ctx, *plan, d_ptr, d_val, cols, d_b, d_c);
    } else if (vec == 2) {
      launch_blocks<2>(ctx, *plan, d_ptr, d_val, cols, d_b, d_c);
    } else {
      launch_blocks<1>(ctx, *plan, d_ptr, d_val, cols, d_b, d_c);
    }
    if (plan->n_direct > 0) {
      spmm_rowsplit_tiles(ctx, n, nnz, d_ptr, d_ind, d_val, cols, d_b, d_c, plan->direct,
                          plan->n_direct, plan->long_rows);
    }
  }
  t.end(ctx.stream);
  ctx.sync();
  if (kernel_ms) *kernel_ms = t.ms();
  t.destroy();
}

} // extern "C"
