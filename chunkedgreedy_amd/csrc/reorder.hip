// reorder.hip -- permutation apply (sporder_reorder).
//
// Reference: sporder/src/reorder.cu:72-149 and bridge sporder/src/sporder.cpp:49-60.
//   ROWS:      ptr_new = scan of gathered row lengths; row p = old row
//              new_order[p] copied verbatim (values alongside).
//   SYMMETRIC: additionally old2new = inverse(new_order), columns mapped
//              through it, and every row re-sorted by column with its values.
//
// The reference sorts rows with cub::DeviceSegmentedSort.  Here rows are
// sorted by size class: up to 64 entries in one wave (register bitonic network
// over lanes), up to kBlockSortCap entries in one workgroup (LDS bitonic), and
// longer rows all together with the library's stable radix sort (by column,
// then by row).  Column
// keys of a valid permutation are distinct within a row, so every method gives
// the same (unique) sorted result.
#include "common.hpp"

#include <algorithm>
#include <vector>

namespace sporder_hip {

namespace {

constexpr int kWaveSortCap = 8 * kWave; // rows sorted in one wave's registers
constexpr int kBlockSortCap = 4096;
constexpr int kBlockSortThreads = 256;
// Rows longer than kBigRow entries are copied by copy_big_rows in units of
// kCopyUnit entries spread over the whole GPU, not by one lane group.
constexpr int kBigRow = 1024;
constexpr int kCopyUnit = 4096;

struct BigRow {
  int32_t src;  // first old entry
  int32_t len;
  int32_t dst;  // first new entry
  int32_t base; // first copy unit
};
struct BigCtl {
  int32_t rows;
  int32_t units;
};

int64_t max_big_rows(int32_t nnz) { return nnz / (kBigRow + 1) + 1; }
int64_t max_copy_units(int32_t nnz) { return nnz / kCopyUnit + max_big_rows(nnz) + 1; }

__global__ void gather_row_lengths(int32_t n, const int32_t *__restrict__ ptr_old,
                                   const int32_t *__restrict__ new2old,
                                   int32_t *__restrict__ ptr_new) {
  for (int64_t p = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
       p < n; p += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int32_t o = new2old[p];
    ptr_new[p + 1] = ptr_old[o + 1] - ptr_old[o];
    if (p == 0) ptr_new[0] = 0;
  }
}

__global__ void invert_perm(int32_t n, const int32_t *__restrict__ src,
                            int32_t *__restrict__ dst) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
       i < n; i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    dst[src[i]] = static_cast<int32_t>(i);
  }
}

// Appends `value` for every lane with `take` to list[*count ...]: one atomic
// per wave, slots in lane order.  Every lane of the wave must call it.
__device__ __forceinline__ void wave_append(bool take, int32_t value, int32_t *list,
                                            int32_t *count) {
  const uint64_t m = ballot(take);
  if (m == 0) return;
  const int leader = __builtin_ctzll(m);
  int32_t base = 0;
  if (lane_id() == leader) base = atomicAdd(count, __popcll(m));
  base = readlane(base, leader);
  if (take) list[base + __popcll(m & ((1ull << lane_id()) - 1ull))] = value;
}

// G lanes per new row (64/G rows per wave).  Copies old row new2old[p] to row
// p, mapping columns through col_map when given.  With col_map (SYMMETRIC) a
// row of at most G entries is also sorted in registers (bitonic network over
// the group's lanes) and written in final order; a longer row is written
// unsorted to key_tmp/val_tmp and appended to the list of the stage that
// sorts it: lists[0] (up to kWaveSortCap entries, sort_rows_wave), lists[1]
// (up to kBlockSortCap, sort_rows_block), lists[2] (longer, the device-wide
// sort), with counts in counts[0..2].  Without col_map (ROWS) rows are copied
// verbatim.  Rows past kBigRow entries are registered for copy_big_rows
// instead of copied here.  All list and registry appends take one atomic per
// wave.  With val_new set and val_old NULL the values written are 0.0f, as in
// the reference's gather_rows (reorder.cu:37-45).
template <int G>
__global__ void __launch_bounds__(256)
    permute_rows(int32_t n, const int32_t *__restrict__ ptr_old,
                 const int32_t *__restrict__ ind_old, const float *__restrict__ val_old,
                 const int32_t *__restrict__ new2old, const int32_t *__restrict__ col_map,
                 const int32_t *__restrict__ ptr_new, int32_t *__restrict__ ind_new,
                 float *__restrict__ val_new, int32_t *__restrict__ key_tmp,
                 float *__restrict__ val_tmp, int32_t *__restrict__ lists,
                 int32_t *__restrict__ counts, int32_t list_stride, BigCtl *big_ctl,
                 BigRow *big_rows, int32_t *big_owner) {
  constexpr int kRowsPerWave = kWave / G;
  const int lane = lane_id();
  const int gl = lane % G;
  const int64_t wave0 = (blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x) / kWave;
  const int64_t nwaves = static_cast<int64_t>(gridDim.x) * blockDim.x / kWave;
  for (int64_t pb = wave0 * kRowsPerWave; pb < n; pb += nwaves * kRowsPerWave) {
    const int64_t p = pb + lane / G;
    const bool row_ok = p < n;
    int32_t src = 0, len = 0, dst = 0;
    if (row_ok) {
      const int32_t o = new2old[p];
      src = ptr_old[o];
      len = ptr_old[o + 1] - src;
      dst = ptr_new[p];
    }
    const bool sort_here = col_map != nullptr && len <= G;
    if (sort_here) {
      const bool in = gl < len;
      int32_t key = in ? col_map[ind_old[src + gl]] : 0x7fffffff;
      float v = (in && val_old) ? val_old[src + gl] : 0.0f;
#pragma unroll
      for (int kk = 2; kk <= G; kk <<= 1) {
#pragma unroll
        for (int j = kk >> 1; j > 0; j >>= 1) {
          const int32_t ok = lane_xor_i32(key, j);
          const float ov = lane_xor_f32(v, j);
          const bool ascending = (gl & kk) == 0;
          const bool lower = (gl & j) == 0;
          if ((ascending == lower) ? (ok < key) : (ok > key)) {
            key = ok;
            v = ov;
          }
        }
      }
      if (in) {
        ind_new[dst + gl] = key;
        if (val_new) val_new[dst + gl] = v;
      }
    } else if (row_ok && len <= kBigRow) {
      int32_t *ki = col_map ? key_tmp : ind_new;
      float *vo = col_map ? val_tmp : val_new;
      // Four entries per lane in flight: the column gather depends on the
      // index load, so one at a time would serialise two latencies per entry.
      for (int32_t q0 = gl; q0 < len; q0 += 4 * G) {
        int32_t c[4];
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int32_t q = q0 + u * G;
          c[u] = q < len ? ind_old[src + q] : 0;
          v[u] = (q < len && val_old) ? val_old[src + q] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int32_t q = q0 + u * G;
          if (q < len) c[u] = col_map ? col_map[c[u]] : c[u];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int32_t q = q0 + u * G;
          if (q < len) {
            ki[dst + q] = c[u];
            if (vo) vo[dst + q] = v[u];
          }
        }
      }
    }
    // Rows sorted here need no bookkeeping; most waves have only those.
    if (ballot(row_ok && !sort_here) == 0) continue;
    // Registry of big rows for copy_big_rows: unit bases from a wave scan.
    const bool big = row_ok && gl == 0 && len > kBigRow;
    const uint64_t mb = ballot(big);
    if (mb != 0) {
      const int32_t units = big ? (len + kCopyUnit - 1) / kCopyUnit : 0;
      const int32_t incl = wave_incl_scan(units);
      const int leader = __builtin_ctzll(mb);
      int32_t rbase = 0, ubase = 0;
      if (lane == leader) {
        rbase = atomicAdd(&big_ctl->rows, __popcll(mb));
        ubase = atomicAdd(&big_ctl->units, readlane(incl, kWave - 1));
      }
      rbase = readlane(rbase, leader);
      ubase = readlane(ubase, leader);
      if (big) {
        const int32_t id = rbase + __popcll(mb & ((1ull << lane) - 1ull));
        const int32_t base = ubase + incl - units;
        big_rows[id] = BigRow{src, len, dst, base};
        for (int32_t u = 0; u < units; ++u) big_owner[base + u] = id;
      }
    }
    if (col_map != nullptr) {
      const bool listed = row_ok && gl == 0 && !sort_here;
      const int32_t row = static_cast<int32_t>(p);
      wave_append(listed && len <= kWaveSortCap, row, lists, counts);
      wave_append(listed && len > kWaveSortCap && len <= kBlockSortCap, row,
                  lists + list_stride, counts + 1);
      wave_append(listed && len > kBlockSortCap, row, lists + 2 * list_stride, counts + 2);
    }
  }
}

// Copy units of the rows registered by permute_rows: a workgroup copies
// kCopyUnit consecutive entries of one row (columns mapped through col_map
// when given), grid-striding over the units.
__global__ void __launch_bounds__(256)
    copy_big_rows(const int32_t *__restrict__ ind_old, const float *__restrict__ val_old,
                  const int32_t *__restrict__ col_map, const BigCtl *__restrict__ big_ctl,
                  const BigRow *__restrict__ big_rows, const int32_t *__restrict__ big_owner,
                  int32_t *__restrict__ ind_out, float *__restrict__ val_out) {
  const int32_t units = big_ctl->units;
  for (int32_t u = blockIdx.x; u < units; u += gridDim.x) {
    const BigRow b = big_rows[big_owner[u]];
    const int32_t q0 = (u - b.base) * kCopyUnit;
    const int32_t q1 = q0 + kCopyUnit < b.len ? q0 + kCopyUnit : b.len;
    for (int32_t q = q0 + static_cast<int32_t>(threadIdx.x); q < q1; q += 256) {
      const int32_t c = ind_old[b.src + q];
      ind_out[b.dst + q] = col_map ? col_map[c] : c;
      if (val_out) val_out[b.dst + q] = val_old ? val_old[b.src + q] : 0.0f;
    }
  }
}

// Bitonic sort of one row of at most 64*P entries held in a wave's registers:
// entry e sits in lane e % 64, register e / 64 (padding keys 0x7fffffff sort
// last; a row's columns are distinct).  Exchanges at distance j < 64 cross
// lanes (lane_xor), longer ones pair registers of the same lane.
template <int P>
__device__ __forceinline__ void wave_sort_row(int32_t s, int32_t len,
                                              const int32_t *__restrict__ key_in,
                                              const float *__restrict__ val_in,
                                              int32_t *__restrict__ key_out,
                                              float *__restrict__ val_out) {
  const int lane = lane_id();
  int32_t key[P];
  float val[P];
#pragma unroll
  for (int r = 0; r < P; ++r) {
    const int32_t e = lane + kWave * r;
    const bool in = e < len;
    key[r] = in ? key_in[s + e] : 0x7fffffff;
    val[r] = (in && val_in) ? val_in[s + e] : 0.0f;
  }
#pragma unroll
  for (int kk = 2; kk <= kWave * P; kk <<= 1) {
#pragma unroll
    for (int j = kk >> 1; j > 0; j >>= 1) {
      if (j >= kWave) {
        const int jr = j / kWave;
#pragma unroll
        for (int r = 0; r < P; ++r) {
          if ((r & jr) == 0) {
            const int q = r | jr;
            const bool asc = ((kWave * r) & kk) == 0; // kk >= 128: lane bits do not matter
            const bool swap = asc ? key[r] > key[q] : key[r] < key[q];
            const int32_t tk = key[r];
            const float tv = val[r];
            key[r] = swap ? key[q] : key[r];
            val[r] = swap ? val[q] : val[r];
            key[q] = swap ? tk : key[q];
            val[q] = swap ? tv : val[q];
          }
        }
      } else {
#pragma unroll
        for (int r = 0; r < P; ++r) {
          const int32_t ok = lane_xor_i32(key[r], j);
          const float ov = lane_xor_f32(val[r], j);
          const bool asc = ((lane + kWave * r) & kk) == 0;
          const bool lower = (lane & j) == 0;
          if ((asc == lower) ? (ok < key[r]) : (ok > key[r])) {
            key[r] = ok;
            val[r] = ov;
          }
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < P; ++r) {
    const int32_t e = lane + kWave * r;
    if (e < len) {
      key_out[s + e] = key[r];
      if (val_out) val_out[s + e] = val[r];
    }
  }
}

// Listed rows of up to kWaveSortCap entries, one wave per row, sorted in
// registers (64, 128, 256 or 512 slots by the row's length; longer rows sort
// faster in a workgroup's LDS).
__global__ void __launch_bounds__(256)
    sort_rows_wave(const int32_t *__restrict__ rows, const int32_t *__restrict__ row_count,
                   const int32_t *__restrict__ ptr, const int32_t *__restrict__ key_in,
                   const float *__restrict__ val_in, int32_t *__restrict__ key_out,
                   float *__restrict__ val_out) {
  const int64_t wave0 = (blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x) / kWave;
  const int64_t nwaves = static_cast<int64_t>(gridDim.x) * blockDim.x / kWave;
  const int64_t count = *row_count;
  for (int64_t t = wave0; t < count; t += nwaves) {
    const int32_t r = rows[t];
    const int32_t s = ptr[r], len = ptr[r + 1] - s;
    if (len <= kWave) {
      wave_sort_row<1>(s, len, key_in, val_in, key_out, val_out);
    } else if (len <= 2 * kWave) {
      wave_sort_row<2>(s, len, key_in, val_in, key_out, val_out);
    } else if (len <= 4 * kWave) {
      wave_sort_row<4>(s, len, key_in, val_in, key_out, val_out);
    } else {
      wave_sort_row<8>(s, len, key_in, val_in, key_out, val_out);
    }
  }
}

// Listed rows of kWaveSortCap+1 .. kBlockSortCap entries: LDS bitonic sort,
// one workgroup per row.
__global__ void __launch_bounds__(kBlockSortThreads)
    sort_rows_block(const int32_t *__restrict__ ptr,
                    const int32_t *__restrict__ long_rows,
                    const int32_t *__restrict__ long_count,
                    const int32_t *__restrict__ key_in,
                    const float *__restrict__ val_in, int32_t *__restrict__ key_out,
                    float *__restrict__ val_out) {
  __shared__ int32_t sk[kBlockSortCap];
  __shared__ float sv[kBlockSortCap];
  const int32_t count = *long_count;
  for (int32_t t = blockIdx.x; t < count; t += gridDim.x) {
    int32_t r = long_rows[t];
    int32_t s = ptr[r], e = ptr[r + 1], len = e - s;
    int32_t pow2 = 1;
    while (pow2 < len) pow2 <<= 1;
    for (int32_t i = threadIdx.x; i < pow2; i += blockDim.x) {
      bool in = i < len;
      sk[i] = in ? key_in[s + i] : 0x7fffffff;
      sv[i] = (in && val_in) ? val_in[s + i] : 0.0f;
    }
    __syncthreads();
    for (int32_t kk = 2; kk <= pow2; kk <<= 1) {
      for (int32_t j = kk >> 1; j > 0; j >>= 1) {
        for (int32_t i = threadIdx.x; i < pow2; i += blockDim.x) {
          int32_t partner = i ^ j;
          if (partner > i) {
            bool ascending = (i & kk) == 0;
            int32_t a = sk[i], b = sk[partner];
            if ((a > b) == ascending) {
              sk[i] = b;
              sk[partner] = a;
              float fa = sv[i];
              sv[i] = sv[partner];
              sv[partner] = fa;
            }
          }
        }
        __syncthreads();
      }
    }
    for (int32_t i = threadIdx.x; i < len; i += blockDim.x) {
      key_out[s + i] = sk[i];
      if (val_out) val_out[s + i] = sv[i];
    }
    __syncthreads();
  }
}

// ---- rows longer than kBlockSortCap: one device-wide sort ------------------
//
// Their entries are gathered into one array and sorted by (row rank, column):
// a stable radix sort by column, then a stable sort by rank, which keeps the
// column order inside each rank.  Rank i's entries then occupy
// [off[i], off[i+1]) in order and are scattered back to row i's range.

__global__ void huge_lengths(const int32_t *__restrict__ ptr_new,
                             const int32_t *__restrict__ huge_rows, int32_t hcount,
                             int32_t *__restrict__ len) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
       i <= hcount; i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    if (i < hcount) {
      const int32_t r = huge_rows[i];
      len[i] = ptr_new[r + 1] - ptr_new[r];
    } else {
      len[i] = 0;
    }
  }
}

// One workgroup per huge row: column keys, gathered indices and ranks.
__global__ void huge_gather(const int32_t *__restrict__ ptr_new,
                            const int32_t *__restrict__ huge_rows, int32_t hcount,
                            const int32_t *__restrict__ off,
                            const int32_t *__restrict__ unsorted,
                            uint32_t *__restrict__ keys, uint32_t *__restrict__ idx,
                            uint32_t *__restrict__ rank) {
  for (int32_t i = blockIdx.x; i < hcount; i += gridDim.x) {
    const int32_t s = ptr_new[huge_rows[i]];
    const int32_t g0 = off[i], len = off[i + 1] - g0;
    for (int32_t t = threadIdx.x; t < len; t += blockDim.x) {
      keys[g0 + t] = static_cast<uint32_t>(unsorted[s + t]);
      idx[g0 + t] = static_cast<uint32_t>(g0 + t);
      rank[g0 + t] = static_cast<uint32_t>(i);
    }
  }
}

__global__ void huge_rank_keys(int64_t count, const uint32_t *__restrict__ by_col,
                               const uint32_t *__restrict__ rank,
                               uint32_t *__restrict__ keys) {
  for (int64_t q = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; q < count;
       q += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    keys[q] = rank[by_col[q]];
  }
}

// Sorted position q holds gathered entry g = order[q] of rank i = rank[g];
// it goes to slot q - off[i] of row huge_rows[i].
__global__ void huge_scatter(int64_t count, const int32_t *__restrict__ ptr_new,
                             const int32_t *__restrict__ huge_rows,
                             const int32_t *__restrict__ off,
                             const uint32_t *__restrict__ order,
                             const uint32_t *__restrict__ rank,
                             const int32_t *__restrict__ unsorted,
                             const float *__restrict__ val_unsorted,
                             int32_t *__restrict__ ind_new, float *__restrict__ val_new) {
  for (int64_t q = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; q < count;
       q += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const uint32_t g = order[q];
    const int32_t i = static_cast<int32_t>(rank[g]);
    const int32_t s = ptr_new[huge_rows[i]];
    const int32_t src = s + static_cast<int32_t>(g) - off[i];
    const int32_t dst = s + static_cast<int32_t>(q) - off[i];
    ind_new[dst] = unsorted[src];
    if (val_new) val_new[dst] = val_unsorted[src];
  }
}

// Sorts rows huge_rows[0 .. hcount) (entries unsorted in `unsorted`,
// `val_unsorted`) into ind_new / val_new.  One host read of the total length.
void sort_huge_rows(Context &ctx, int32_t n, const int32_t *ptr_new, const int32_t *huge_rows,
                    int32_t hcount, const int32_t *unsorted, const float *val_unsorted,
                    int32_t *ind_new, float *val_new, int32_t *off, int32_t *scan_tmp) {
  const int g1 = ctx.grid_for(ceil_div64(static_cast<int64_t>(hcount) + 1, 256), 256, 4);
  huge_lengths<<<g1, 256, 0, ctx.stream>>>(ptr_new, huge_rows, hcount, off);
  SP_LAUNCH_CHECK();
  scan_i32(ctx, off, off, static_cast<int64_t>(hcount) + 1, false, scan_tmp);
  int32_t total = 0;
  SP_HIP(hipMemcpyAsync(&total, off + hcount, sizeof(int32_t), hipMemcpyDeviceToHost,
                        ctx.stream));
  ctx.sync();
  if (total == 0) return;
  const size_t H = static_cast<size_t>(total);
  const size_t tmp_elems = radix_tmp_elems(total);
  auto *base = static_cast<uint32_t *>(ctx.aux_reserve((7 * H + tmp_elems) * 4 + 8 * 256));
  auto carve = [&](size_t elems) {
    uint32_t *p = base;
    base += (elems + 63) & ~size_t(63);
    return p;
  };
  uint32_t *keys = carve(H), *idx = carve(H), *rank = carve(H), *k1 = carve(H), *v1 = carve(H);
  uint32_t *ka = carve(H), *va = carve(H);
  int32_t *tmp = reinterpret_cast<int32_t *>(carve(tmp_elems));
  huge_gather<<<std::min<int32_t>(hcount, ctx.num_cus * 8), 256, 0, ctx.stream>>>(
      ptr_new, huge_rows, hcount, off, unsorted, keys, idx, rank);
  SP_LAUNCH_CHECK();
  radix_sort_pairs(ctx, keys, idx, k1, v1, ka, va, total, bits_for(n - 1), tmp);
  const int gq = ctx.grid_for(ceil_div64(total, 256), 256, 4);
  huge_rank_keys<<<gq, 256, 0, ctx.stream>>>(total, v1, rank, keys);
  SP_LAUNCH_CHECK();
  radix_sort_pairs(ctx, keys, v1, k1, idx, ka, va, total, bits_for(hcount - 1), tmp);
  huge_scatter<<<gq, 256, 0, ctx.stream>>>(total, ptr_new, huge_rows, off, idx, rank, unsorted,
                                           val_unsorted, ind_new, val_new);
  SP_LAUNCH_CHECK();
}

template <int G>
void launch_permute_g(Context &ctx, int32_t n, const int32_t *ptr_old, const int32_t *ind_old,
                      const float *val_old, const int32_t *new2old, const int32_t *col_map,
                      const int32_t *ptr_new, int32_t *ind_new, float *val_new,
                      int32_t *key_tmp, float *val_tmp, int32_t *lists, int32_t *counts,
                      int32_t list_stride, BigCtl *big_ctl, BigRow *big_rows,
                      int32_t *big_owner) {
  constexpr int rows_per_block = 4 * (kWave / G);
  const int g = ctx.grid_for(ceil_div64(n, rows_per_block), 256, 4);
  permute_rows<G><<<g, 256, 0, ctx.stream>>>(n, ptr_old, ind_old, val_old, new2old, col_map,
                                            ptr_new, ind_new, val_new, key_tmp, val_tmp,
                                            lists, counts, list_stride, big_ctl, big_rows,
                                            big_owner);
  SP_LAUNCH_CHECK();
}

void launch_permute(Context &ctx, int G, int32_t n, const int32_t *ptr_old,
                    const int32_t *ind_old, const float *val_old, const int32_t *new2old,
                    const int32_t *col_map, const int32_t *ptr_new, int32_t *ind_new,
                    float *val_new, int32_t *key_tmp, float *val_tmp, int32_t *lists,
                    int32_t *counts, int32_t list_stride, int32_t nnz, BigCtl *big_ctl,
                    BigRow *big_rows, int32_t *big_owner) {
  fill_u32(ctx, big_ctl, sizeof(BigCtl) / 4, 0u);
  switch (G) {
#define SP_CASE(V)                                                                       \
  case V:                                                                                \
    launch_permute_g<V>(ctx, n, ptr_old, ind_old, val_old, new2old, col_map, ptr_new,    \
                        ind_new, val_new, key_tmp, val_tmp, lists, counts, list_stride,  \
                        big_ctl, big_rows, big_owner);                                   \
    break;
    SP_CASE(4) SP_CASE(8) SP_CASE(16) SP_CASE(32) SP_CASE(64)
#undef SP_CASE
  default:
    SP_EXPECT(false, "internal: bad group width");
  }
  // Big rows' units (none registered: every workgroup exits at once).
  const int gb = ctx.grid_for(max_copy_units(nnz), 256, 4);
  copy_big_rows<<<gb, 256, 0, ctx.stream>>>(ind_old, val_old, col_map, big_ctl, big_rows,
                                            big_owner, col_map ? key_tmp : ind_new,
                                            col_map ? val_tmp : val_new);
  SP_LAUNCH_CHECK();
}

} // namespace

} // namespace sporder_hip

using namespace sporder_hip;

extern "C" void sporder_reorder(sporder_context_t h, int32_t n, int32_t nnz,
                                const int32_t *d_ptr_old, const int32_t *d_ind_old,
                                const float *d_val_old, const int32_t *d_new_order,
                                sporder_reorder_mode_t mode, int32_t *d_ptr_new,
                                int32_t *d_ind_new, float *d_val_new) {
  SP_EXPECT(h != nullptr, "null context");
  SP_EXPECT(mode == SPORDER_REORDER_ROWS || mode == SPORDER_REORDER_SYMMETRIC,
            "invalid reorder mode");
  SP_EXPECT(n >= 1 && nnz >= 0, "expect n >= 1 and nnz >= 0");
  Context &ctx = h->impl;
  const bool symmetric = mode == SPORDER_REORDER_SYMMETRIC;
  const bool with_vals = d_val_old != nullptr && d_val_new != nullptr;

  size_t need = ws_bytes<int32_t>(scan_tmp_elems(static_cast<int64_t>(n) + 1)) +
                ws_bytes<BigCtl>(1) + ws_bytes<BigRow>(static_cast<size_t>(max_big_rows(nnz))) +
                ws_bytes<int32_t>(static_cast<size_t>(max_copy_units(nnz)));
  if (symmetric) {
    need += ws_bytes<int32_t>(n) + ws_bytes<int32_t>(nnz) + ws_bytes<float>(nnz) +
            ws_bytes<int32_t>(3 * (static_cast<size_t>(n) + 2)) + ws_bytes<int32_t>(3);
  }
  ctx.reserve(need);
  int32_t *scan_tmp = ctx.take<int32_t>(scan_tmp_elems(static_cast<int64_t>(n) + 1));
  BigCtl *big_ctl = ctx.take<BigCtl>(1);
  BigRow *big_rows = ctx.take<BigRow>(static_cast<size_t>(max_big_rows(nnz)));
  int32_t *big_owner = ctx.take<int32_t>(static_cast<size_t>(max_copy_units(nnz)));

  const int row_grid = ctx.grid_for(ceil_div64(n, 256), 256, 4);
  const int wave_grid = ctx.grid_for(ceil_div64(n, 4), 256, 4);

  gather_row_lengths<<<row_grid, 256, 0, ctx.stream>>>(n, d_ptr_old, d_new_order,
                                                       d_ptr_new);
  SP_LAUNCH_CHECK();
  scan_i32(ctx, d_ptr_new, d_ptr_new, static_cast<int64_t>(n) + 1, true, scan_tmp);

  // Lanes per row: the average row length rounded up to a power of two,
  // between 4 and 64.
  int G = 4;
  while (G < 64 && static_cast<int64_t>(G) * n < nnz) G <<= 1;

  if (!symmetric) {
    launch_permute(ctx, G, n, d_ptr_old, d_ind_old, d_val_old, d_new_order, nullptr,
                   d_ptr_new, d_ind_new, d_val_new, nullptr, nullptr, nullptr, nullptr, 0, nnz,
                   big_ctl, big_rows, big_owner);
    ctx.sync();
    return;
  }

  int32_t *old2new = ctx.take<int32_t>(n);
  int32_t *unsorted = ctx.take<int32_t>(nnz);
  float *val_unsorted = ctx.take<float>(nnz);
  // Row lists of the three sort stages, one array with stride n + 2.
  const int32_t stride = n + 2;
  int32_t *lists = ctx.take<int32_t>(3 * static_cast<size_t>(stride));
  int32_t *list1 = lists, *long_rows = lists + stride, *huge_rows = lists + 2 * stride;
  int32_t *counts = ctx.take<int32_t>(3);

  invert_perm<<<row_grid, 256, 0, ctx.stream>>>(n, d_new_order, old2new);
  SP_LAUNCH_CHECK();
  fill_u32(ctx, counts, 3, 0u);
  // Rows of at most G entries are remapped, sorted and written in one pass;
  // longer rows are written unsorted to the temporaries and listed by length
  // for the stage that sorts them.
  launch_permute(ctx, G, n, d_ptr_old, d_ind_old, d_val_old, d_new_order, old2new,
                 d_ptr_new, d_ind_new, with_vals ? d_val_new : nullptr, unsorted,
                 with_vals ? val_unsorted : nullptr, lists, counts, stride, nnz, big_ctl,
                 big_rows, big_owner);
  sort_rows_wave<<<wave_grid, 256, 0, ctx.stream>>>(
      list1, counts, d_ptr_new, unsorted, with_vals ? val_unsorted : nullptr, d_ind_new,
      with_vals ? d_val_new : nullptr);
  SP_LAUNCH_CHECK();
  sort_rows_block<<<ctx.num_cus * 4, kBlockSortThreads, 0, ctx.stream>>>(
      d_ptr_new, long_rows, counts + 1, unsorted, with_vals ? val_unsorted : nullptr,
      d_ind_new, with_vals ? d_val_new : nullptr);
  SP_LAUNCH_CHECK();

  int32_t hcount = 0;
  SP_HIP(hipMemcpyAsync(&hcount, counts + 2, sizeof(int32_t), hipMemcpyDeviceToHost,
                        ctx.stream));
  ctx.sync();
  if (hcount > 0) {
    sort_huge_rows(ctx, n, d_ptr_new, huge_rows, hcount, unsorted,
                   with_vals ? val_unsorted : nullptr, d_ind_new,
                   with_vals ? d_val_new : nullptr, list1, scan_tmp);
  }
  ctx.sync();
}
