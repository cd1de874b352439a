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
#include <cstring>
#include <vector>

namespace sporder_hip {

namespace {

constexpr int kWaveSortCap = 8 * kWave; // rows sorted in one wave's registers
constexpr int kBlockSortCap = 4096;
constexpr int kBlockSortThreads = 256;
// Rows longer than kBigRow entries are copied by copy_big_rows in units of
// kCopyUnit entries spread over the whole GPU, not by one lane group.
constexpr int kBigRow = 1024;
constexpr int kPrepBlock = 1024;
constexpr int kCopyUnit = 4096;
// sort_runs: blocks of up to 2^kRunMaxBits columns (a bitmap of that many
// bits per wave in LDS); runs of at most kRunRankCap entries are placed by
// counting, in registers.
constexpr int kRunMaxBits = 13;
constexpr int kRunWords = (1 << kRunMaxBits) / 32;
constexpr int kRunBlock = 256;
constexpr int kRunWaves = kRunBlock / kWave;
constexpr int kRunRankCap = 8;

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
// One call's control words, zeroed by prepare_rows and read back after
// permute_rows (and after sort_runs): the three sort-list counts, the big-row
// registry's counts, the wide-remap flag, the bit count `sh` of the largest
// c ^ old2new[c] (every column stays inside its aligned block of 2^sh), and
// the flag sort_runs sets when an input row is not strictly increasing.
struct Ctl {
  int32_t counts[3];
  BigCtl big;
  int32_t wide;
  int32_t sh;
  int32_t unsorted;
};
// Words of Ctl that a second permute_rows pass appends to from zero.
constexpr int kCtlListWords = 5;

int64_t max_big_rows(int32_t nnz) { return nnz / (kBigRow + 1) + 1; }
int64_t max_copy_units(int32_t nnz) { return nnz / kCopyUnit + max_big_rows(nnz) + 1; }

// Per new row p, with o = new2old[p]: src_new[p] = ptr_old[o] (where the old
// row starts), ptr_new[p + 1] = the row's length (ptr_new[0] = 0, so an
// inclusive scan gives the offsets) and, when old2new is given, old2new[o] = p.
// Doing the two dependent loads here leaves permute_rows one coalesced load
// before its row gathers.  One workgroup per scan tile of ptr_new (elements
// [t * kScanTileElems, (t + 1) * kScanTileElems), element i = p + 1), whose
// sum goes to totals[t], so the scan starts at its second pass.  Block 0 also
// zeroes the call's control words.
__global__ void __launch_bounds__(kPrepBlock)
    prepare_rows(int32_t n, const int32_t *__restrict__ ptr_old,
                 const int32_t *__restrict__ new2old, int32_t *__restrict__ ptr_new,
                 int32_t *__restrict__ src_new, int32_t *__restrict__ old2new,
                 int32_t *__restrict__ totals, Ctl *__restrict__ ctl) {
  __shared__ int32_t s_wave[kPrepBlock / kWave];
  if (blockIdx.x == 0 && threadIdx.x < sizeof(Ctl) / 4) {
    reinterpret_cast<int32_t *>(ctl)[threadIdx.x] = 0;
  }
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTileElems;
  int32_t sum = 0;
#pragma unroll 4
  for (int r = 0; r < kScanTileElems / kPrepBlock; ++r) {
    const int64_t i = base + r * kPrepBlock + threadIdx.x;
    if (i == 0) {
      ptr_new[0] = 0;
    } else if (i <= n) {
      const int64_t p = i - 1;
      const int32_t o = new2old[p];
      const int32_t s = ptr_old[o];
      const int32_t len = ptr_old[o + 1] - s;
      src_new[p] = s;
      ptr_new[i] = len;
      if (old2new) old2new[o] = static_cast<int32_t>(p);
      sum += len;
    }
  }
  sum = wave_sum(sum);
  if (lane_id() == 0) s_wave[threadIdx.x / kWave] = sum;
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t t = 0;
#pragma unroll
    for (int w = 0; w < kPrepBlock / kWave; ++w) t += s_wave[w];
    totals[blockIdx.x] = t;
  }
}

// delta[c] = old2new[c] - c as 16 bits, for the column remap: a permutation
// that moves every index by less than 2^15 (csg's, whose chains stay inside
// chunks of at most 32768 rows, among them) gets a table half the size of
// old2new, which stays in L2 where the 4-byte table at n = 2^20 fills it.  Any
// larger move sets ctl->wide, and permute_rows then reads old2new.  Also
// ctl->sh = the bit length of the largest c ^ old2new[c]: every column then
// stays inside its aligned block of 2^sh indices (c >> sh is unchanged), which
// is what lets sort_runs sort only within blocks (csg's chunk-local orders
// give sh <= log2(chunk_size) for a power-of-two chunk size).
__global__ void __launch_bounds__(256)
    narrow_map(int32_t n, const int32_t *__restrict__ old2new, int16_t *__restrict__ delta,
               Ctl *__restrict__ ctl) {
  __shared__ int32_t s_far, s_sh;
  if (threadIdx.x == 0) {
    s_far = 0;
    s_sh = 0;
  }
  __syncthreads();
  bool far = false;
  uint32_t moved = 0; // OR of c ^ old2new[c]: its bit length is the largest one's
  for (int64_t c = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; c < n;
       c += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int32_t o = old2new[c];
    const int32_t d = o - static_cast<int32_t>(c);
    far |= d < -32768 || d > 32767;
    moved |= static_cast<uint32_t>(o) ^ static_cast<uint32_t>(c);
    delta[c] = static_cast<int16_t>(d);
  }
  if (far) s_far = 1;
  const int32_t sh = moved ? 32 - __clz(static_cast<int32_t>(moved)) : 0;
  const int32_t wsh = static_cast<int32_t>(wave_max_u32(static_cast<uint32_t>(sh)));
  if (lane_id() == 0 && wsh != 0) atomicMax(&s_sh, wsh);
  __syncthreads();
  // One atomic per workgroup (the grid is a few per CU): a random permutation
  // sets the flag from every workgroup, and per-wave atomics on one word
  // would serialise.
  if (threadIdx.x == 0 && s_far != 0) atomicOr(&ctl->wide, 1);
  if (threadIdx.x == 0 && s_sh != 0) atomicMax(&ctl->sh, s_sh);
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

// Bitonic sort, ascending by key, of the G entries held one per lane by a
// group of G lanes (gl = lane within the group; padding keys 0x7fffffff).
template <int G>
__device__ __forceinline__ void group_sort(int32_t &key, float &v, int gl) {
#pragma unroll
  for (int kk = 2; kk <= G; kk <<= 1) {
#pragma unroll
    for (int j = kk >> 1; j > 0; j >>= 1) {
      const bool ascending = (gl & kk) == 0;
      const bool lower = (gl & j) == 0;
      const int32_t ok = lane_xor_i32(key, j);
      const float ov = lane_xor_f32(v, j);
      if ((ascending == lower) ? (ok < key) : (ok > key)) {
        key = ok;
        v = ov;
      }
    }
  }
}

// The same for 2G entries, entry e = gl + G * r in register r (0: key/v,
// 1: key2/v2): exchanges at distance G are between a lane's two registers,
// shorter ones across lanes.
template <int G>
__device__ __forceinline__ void group_sort2(int32_t &key, float &v, int32_t &key2, float &v2,
                                            int gl) {
#pragma unroll
  for (int kk = 2; kk <= 2 * G; kk <<= 1) {
#pragma unroll
    for (int j = kk >> 1; j > 0; j >>= 1) {
      if (j == G) { // kk == 2G: every pair ascending
        if (key2 < key) {
          const int32_t tk = key;
          key = key2;
          key2 = tk;
          const float tv = v;
          v = v2;
          v2 = tv;
        }
        continue;
      }
      const bool lower = (gl & j) == 0;
      const bool asc0 = (gl & kk) == 0, asc1 = ((gl + G) & kk) == 0;
      const int32_t ok = lane_xor_i32(key, j), ok2 = lane_xor_i32(key2, j);
      const float ov = lane_xor_f32(v, j), ov2 = lane_xor_f32(v2, j);
      if ((asc0 == lower) ? (ok < key) : (ok > key)) {
        key = ok;
        v = ov;
      }
      if ((asc1 == lower) ? (ok2 < key2) : (ok2 > key2)) {
        key2 = ok2;
        v2 = ov2;
      }
    }
  }
}

// G lanes per new row; a wave takes U groups of 64/G rows per iteration, and
// their loads are issued together, so U gather chains (row entries, then the
// column map) are in flight per wave instead of one.  Copies old row
// new2old[p] (which starts at src_new[p]) to row p, mapping columns through
// col_map when given.  With col_map (SYMMETRIC) a row of at most 2G entries is
// also sorted in registers (bitonic network over the group's lanes, one or two
// registers each) and written in final order; a longer row is appended to the
// list of the stage that sorts it, with counts in ctl->counts[0..2]: lists[0]
// (up to kWaveSortCap entries, sort_rows_wave, which reads the row written
// here unsorted to key_tmp/val_tmp), lists[1] (up to kBlockSortCap,
// sort_rows_block, which gathers the old row itself), lists[2] (longer, the
// device-wide sort, whose rows are registered for copy_big_rows).  Without
// col_map (ROWS) rows are copied verbatim, and rows past kBigRow entries are
// registered for copy_big_rows.  List and registry appends take one atomic
// per wave that has such rows: rows past 2G entries are a minority even on
// power-law inputs, while a list of every row past G entries (a fifth of the
// rows of a mean-13 random geometric graph) serialised on its counter.  With
// val_new set and val_old NULL the values written are 0.0f, as in the
// reference's gather_rows (reorder.cu:37-45).
template <int G, int U>
__global__ void __launch_bounds__(256)
    permute_rows(int32_t n, const int32_t *__restrict__ src_new,
                 const int32_t *__restrict__ ind_old, const float *__restrict__ val_old,
                 const int32_t *__restrict__ col_map, const int16_t *__restrict__ delta,
                 const int32_t *__restrict__ ptr_new,
                 int32_t *__restrict__ ind_new, float *__restrict__ val_new,
                 int32_t *__restrict__ key_tmp, float *__restrict__ val_tmp,
                 int32_t *__restrict__ lists, int32_t list_stride, Ctl *__restrict__ ctl,
                 BigRow *big_rows, int32_t *big_owner, int allow_runs) {
  constexpr int kRowsPerWave = kWave / G;
  // The 16-bit remap when narrow_map found every move within its range.
  const bool narrow = delta != nullptr && ctl->wide == 0;
  // Run mode: the listed rows are gathered and sorted by sort_runs itself,
  // so they are not copied here.
  const bool runs = narrow && allow_runs != 0 && ctl->sh <= kRunMaxBits;
  constexpr int kRowsPerIter = kRowsPerWave * U;
  const int lane = lane_id();
  const int gl = lane % G;
  const int64_t wave0 = (blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x) / kWave;
  const int64_t nwaves = static_cast<int64_t>(gridDim.x) * blockDim.x / kWave;
  for (int64_t pb = wave0 * kRowsPerIter; pb < n; pb += nwaves * kRowsPerIter) {
    int32_t src[U], len[U], dst[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t p = pb + u * kRowsPerWave + lane / G;
      const bool ok = p < n;
      src[u] = ok ? src_new[p] : 0;
      dst[u] = ok ? ptr_new[p] : 0;
      len[u] = ok ? ptr_new[p + 1] - dst[u] : 0;
    }
    if (col_map != nullptr) {
      // Rows of at most 2G entries: gather, remap, sort, store.  Lane gl of
      // a row's group holds entries gl and gl + G; a group of rows none of
      // which passes G entries sorts the first register only.
      int32_t key[U], key2[U];
      float v[U], v2[U];
      bool wide2[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool fits = len[u] <= 2 * G;
        const bool in = gl < len[u] && fits, in2 = gl + G < len[u] && fits;
        key[u] = in ? ind_old[src[u] + gl] : 0;
        v[u] = (in && val_old) ? val_old[src[u] + gl] : 0.0f;
        key2[u] = in2 ? ind_old[src[u] + gl + G] : 0;
        v2[u] = (in2 && val_old) ? val_old[src[u] + gl + G] : 0.0f;
        wide2[u] = ballot(len[u] > G && fits) != 0;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool fits = len[u] <= 2 * G;
        const bool in = gl < len[u] && fits, in2 = gl + G < len[u] && fits;
        if (narrow) {
          key[u] = in ? key[u] + delta[key[u]] : 0x7fffffff;
          key2[u] = in2 ? key2[u] + delta[key2[u]] : 0x7fffffff;
        } else {
          key[u] = in ? col_map[key[u]] : 0x7fffffff;
          key2[u] = in2 ? col_map[key2[u]] : 0x7fffffff;
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (wide2[u]) {
          group_sort2<G>(key[u], v[u], key2[u], v2[u], gl);
        } else {
          group_sort<G>(key[u], v[u], gl);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool fits = len[u] <= 2 * G;
        if (gl < len[u] && fits) {
          __builtin_nontemporal_store(key[u], ind_new + dst[u] + gl);
          if (val_new) __builtin_nontemporal_store(v[u], val_new + dst[u] + gl);
        }
        if (gl + G < len[u] && fits) {
          __builtin_nontemporal_store(key2[u], ind_new + dst[u] + gl + G);
          if (val_new) __builtin_nontemporal_store(v2[u], val_new + dst[u] + gl + G);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t p = pb + u * kRowsPerWave + lane / G;
      const bool row_ok = p < n;
      const bool sort_here = col_map != nullptr && len[u] <= 2 * G;
      // Rows sorted above need no bookkeeping; most waves have only those.
      if (ballot(row_ok && !sort_here) == 0) continue;
      const int32_t copy_cap = col_map ? kWaveSortCap : kBigRow;
      if (row_ok && !sort_here && len[u] <= copy_cap && !runs) {
        int32_t *ki = col_map ? key_tmp : ind_new;
        float *vo = col_map ? val_tmp : val_new;
        // Four entries per lane in flight: the column gather depends on the
        // index load, so one at a time would serialise two latencies per entry.
        for (int32_t q0 = gl; q0 < len[u]; q0 += 4 * G) {
          int32_t c[4];
          float w[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int32_t q = q0 + t * G;
            c[t] = q < len[u] ? ind_old[src[u] + q] : 0;
            w[t] = (q < len[u] && val_old) ? val_old[src[u] + q] : 0.0f;
          }
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int32_t q = q0 + t * G;
            if (q < len[u]) {
              c[t] = narrow ? c[t] + delta[c[t]] : (col_map ? col_map[c[t]] : c[t]);
            }
          }
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int32_t q = q0 + t * G;
            if (q < len[u]) {
              ki[dst[u] + q] = c[t];
              if (vo) vo[dst[u] + q] = w[t];
            }
          }
        }
      }
      // Registry of big rows for copy_big_rows: unit bases from a wave scan.
      const bool big = row_ok && gl == 0 && len[u] > (col_map ? kBlockSortCap : kBigRow);
      const uint64_t mb = ballot(big);
      if (mb != 0) {
        const int32_t units = big ? (len[u] + kCopyUnit - 1) / kCopyUnit : 0;
        const int32_t incl = wave_incl_scan(units);
        const int leader = __builtin_ctzll(mb);
        int32_t rbase = 0, ubase = 0;
        if (lane == leader) {
          rbase = atomicAdd(&ctl->big.rows, __popcll(mb));
          ubase = atomicAdd(&ctl->big.units, readlane(incl, kWave - 1));
        }
        rbase = readlane(rbase, leader);
        ubase = readlane(ubase, leader);
        if (big) {
          const int32_t id = rbase + __popcll(mb & ((1ull << lane) - 1ull));
          const int32_t base = ubase + incl - units;
          big_rows[id] = BigRow{src[u], len[u], dst[u], base};
          for (int32_t k = 0; k < units; ++k) big_owner[base + k] = id;
        }
      }
      if (col_map != nullptr) {
        const bool listed = row_ok && gl == 0 && !sort_here;
        const int32_t row = static_cast<int32_t>(p);
        wave_append(listed && len[u] <= kWaveSortCap, row, lists, ctl->counts);
        wave_append(listed && len[u] > kWaveSortCap && len[u] <= kBlockSortCap, row,
                    lists + list_stride, ctl->counts + 1);
        wave_append(listed && len[u] > kBlockSortCap, row, lists + 2 * list_stride,
                    ctl->counts + 2);
      }
    }
  }
}

// Copy units of the rows registered by permute_rows: a workgroup copies
// kCopyUnit consecutive entries of one row (columns mapped through col_map
// when given), grid-striding over the units.
__global__ void __launch_bounds__(256)
    copy_big_rows(const int32_t *__restrict__ ind_old, const float *__restrict__ val_old,
                  const int32_t *__restrict__ col_map, int32_t units,
                  const BigRow *__restrict__ big_rows, const int32_t *__restrict__ big_owner,
                  int32_t *__restrict__ ind_out, float *__restrict__ val_out) {
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
    sort_rows_wave(const int32_t *__restrict__ rows, int32_t count,
                   const int32_t *__restrict__ ptr, const int32_t *__restrict__ key_in,
                   const float *__restrict__ val_in, int32_t *__restrict__ key_out,
                   float *__restrict__ val_out) {
  const int64_t wave0 = (blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x) / kWave;
  const int64_t nwaves = static_cast<int64_t>(gridDim.x) * blockDim.x / kWave;
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

// Listed rows of kWaveSortCap+1 .. kBlockSortCap entries, one workgroup per
// row: the old row (starting at src_new[r]) is gathered with its columns
// remapped (the 16-bit delta table when `narrow`, else col_map), sorted in
// LDS (bitonic) and written to row r.
__global__ void __launch_bounds__(kBlockSortThreads)
    sort_rows_block(const int32_t *__restrict__ ptr, const int32_t *__restrict__ long_rows,
                    int32_t long_count, const int32_t *__restrict__ src_new,
                    const int32_t *__restrict__ ind_old, const float *__restrict__ val_old,
                    const int32_t *__restrict__ col_map, const int16_t *__restrict__ delta,
                    bool narrow, int32_t *__restrict__ key_out, float *__restrict__ val_out) {
  __shared__ int32_t sk[kBlockSortCap];
  __shared__ float sv[kBlockSortCap];
  for (int32_t t = blockIdx.x; t < long_count; t += gridDim.x) {
    const int32_t r = long_rows[t];
    const int32_t s = ptr[r], len = ptr[r + 1] - s, src = src_new[r];
    int32_t pow2 = 1;
    while (pow2 < len) pow2 <<= 1;
    for (int32_t i = threadIdx.x; i < pow2; i += blockDim.x) {
      const bool in = i < len;
      const int32_t c = in ? ind_old[src + i] : 0;
      sk[i] = in ? (narrow ? c + delta[c] : col_map[c]) : 0x7fffffff;
      sv[i] = (in && val_old) ? val_old[src + i] : 0.0f;
    }
    __syncthreads();
    for (int32_t kk = 2; kk <= pow2; kk <<= 1) {
      for (int32_t j = kk >> 1; j > 0; j >>= 1) {
        for (int32_t i = threadIdx.x; i < pow2; i += blockDim.x) {
          const int32_t partner = i ^ j;
          if (partner > i) {
            const bool ascending = (i & kk) == 0;
            const int32_t a = sk[i], b = sk[partner];
            if ((a > b) == ascending) {
              sk[i] = b;
              sk[partner] = a;
              const float fa = sv[i];
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

// ---- run mode: rows already ordered by block ---------------------------------
//
// When every column c stays inside its aligned block of 2^sh indices
// (old2new[c] >> sh == c >> sh) and an input row is strictly increasing, the
// remapped row is already ordered by block: it is a sequence of runs of
// entries with equal c >> sh, and sorting it means sorting each run on its
// own.  A run holds at most 2^sh entries (distinct columns of one block), and
// its remapped columns have distinct low sh bits.
//
// sort_runs gives each wave one task: a whole listed row of at most
// kBlockSortCap entries, or one kCopyUnit-entry unit of a longer row (the
// units permute_rows registered), widened at both ends to the next run
// boundary so that every run belongs to exactly one task.  The wave walks its
// range 64 entries at a time:
//   - the longest prefix of whole runs inside the window is placed at once:
//     singleton runs are copied, runs of at most kRunRankCap entries are
//     placed by counting the smaller keys of their run (shuffles), otherwise
//     the prefix is sorted by a bitonic network over the wave (it consists of
//     whole runs, so sorting it by remapped column sorts each run);
//   - a run longer than the window is placed with a bitmap of its low bits
//     in LDS: one pass sets a bit per entry, a scan of the words' population
//     counts gives each word's rank, a second pass writes each entry at its
//     rank.
// Every pair of neighbouring input entries of the task is checked; a row
// that is not strictly increasing sets ctl->unsorted, and the host then
// redoes the call's long rows with the full sorts (positions stay inside the
// task's output range either way).

struct RunBits {
  uint32_t bits[kRunWords];
  uint32_t rank[kRunWords];
};

// First index i >= q with i == len or c[i] >> sh != c[i - 1] >> sh (q >= 1):
// a run boundary.  For a strictly increasing row it lies within 2^sh entries
// of q; a longer search means the row is not, and sets *bad (the result is
// then any deterministic index in [q, len], the same for both tasks that ask).
__device__ __forceinline__ int32_t next_run_start(const int32_t *__restrict__ row, int32_t q,
                                                  int32_t len, int sh, bool *bad) {
  const int lane = lane_id();
  for (int32_t w0 = q; w0 < len; w0 += kWave) {
    const int32_t i = w0 + lane;
    bool edge = i >= len;
    if (!edge) edge = (row[i] >> sh) != (row[i - 1] >> sh);
    const uint64_t m = ballot(edge);
    if (m != 0) return w0 + __builtin_ctzll(m);
    if (w0 + kWave - q > (1 << sh)) {
      *bad = true;
      return w0 + kWave < len ? w0 + kWave : len;
    }
  }
  return len;
}

// Places the run starting at s (longer than one window) through the wave's
// bitmap; returns its end.  Entries past the run (another block) are left to
// the caller.
__device__ __forceinline__ int32_t place_long_run(RunBits *rb, const int32_t *__restrict__ ind,
                                                  const float *__restrict__ val,
                                                  const int16_t *__restrict__ delta, int32_t s,
                                                  int32_t b, int32_t len, int sh,
                                                  int32_t *__restrict__ key_out,
                                                  float *__restrict__ val_out, bool *bad) {
  const int lane = lane_id();
  const int32_t h0 = ind[s] >> sh;
  const uint32_t lowmask = (1u << sh) - 1u;
  const int words = sh >= 5 ? (1 << (sh - 5)) : 1;
  int32_t re = b;
  for (int32_t w0 = s;; w0 += kWave) {
    const int32_t i = w0 + lane;
    const bool in = i < b;
    const int32_t c = in ? ind[i] : 0;
    const bool inrun = in && (c >> sh) == h0;
    if (inrun) {
      const int32_t cn = i + 1 < len ? ind[i + 1] : 0x7fffffff;
      if (cn <= c) *bad = true;
      const uint32_t low = static_cast<uint32_t>(c + delta[c]) & lowmask;
      atomicOr(&rb->bits[low >> 5], 1u << (low & 31u));
    }
    const int cnt = __popcll(ballot(inrun));
    if (cnt < kWave) {
      re = w0 + cnt;
      break;
    }
    if (w0 + kWave - s > (1 << sh)) {
      // More than 2^sh entries of one block: not strictly increasing.
      *bad = true;
      re = w0 + kWave;
      break;
    }
  }
  wave_lds_order();
  // Rank of each word: the set bits of the words before it.
  int32_t carry = 0;
  for (int w = lane; w - lane < words; w += kWave) {
    const int32_t x = w < words ? __popc(rb->bits[w]) : 0;
    const int32_t incl = wave_incl_scan(x);
    if (w < words) rb->rank[w] = carry + incl - x;
    carry += readlane(incl, kWave - 1);
  }
  wave_lds_order();
  for (int32_t w0 = s; w0 < re; w0 += kWave) {
    const int32_t i = w0 + lane;
    if (i < re) {
      const int32_t c = ind[i];
      // Entries of another block (only in a row that is not strictly
      // increasing) are not written: their bit may be missing.
      if ((c >> sh) == h0) {
        const int32_t key = c + delta[c];
        const uint32_t low = static_cast<uint32_t>(key) & lowmask;
        const uint32_t word = rb->bits[low >> 5];
        const int32_t pos = rb->rank[low >> 5] + __popc(word & ((1u << (low & 31u)) - 1u));
        key_out[s + pos] = key;
        if (val_out) val_out[s + pos] = val ? val[i] : 0.0f;
      }
    }
  }
  wave_lds_order();
  for (int w = lane; w < words; w += kWave) rb->bits[w] = 0;
  wave_lds_order();
  return re;
}

__global__ void __launch_bounds__(kRunBlock)
    sort_runs(const int32_t *__restrict__ lists, int32_t list_stride, int32_t rows0,
              int32_t rows1, int32_t units, const int32_t *__restrict__ ptr_new,
              const int32_t *__restrict__ src_new, const BigRow *__restrict__ big_rows,
              const int32_t *__restrict__ big_owner, const int32_t *__restrict__ ind_old,
              const float *__restrict__ val_old, const int16_t *__restrict__ delta, int sh,
              int32_t *__restrict__ ind_new, float *__restrict__ val_new,
              Ctl *__restrict__ ctl) {
  __shared__ RunBits s_bits[kRunWaves];
  RunBits *rb = &s_bits[threadIdx.x / kWave];
  const int lane = lane_id();
  for (int w = lane; w < kRunWords; w += kWave) rb->bits[w] = 0;
  wave_lds_order();
  bool bad = false;
  const int64_t wave0 = (blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x) / kWave;
  const int64_t nwaves = static_cast<int64_t>(gridDim.x) * blockDim.x / kWave;
  const int64_t tasks = static_cast<int64_t>(units) + rows1 + rows0;
  // Units (the longest rows) first, then the rows of the two lists.
  for (int64_t t = wave0; t < tasks; t += nwaves) {
    int32_t src, len, dst, a, b;
    if (t < units) {
      const BigRow br = big_rows[big_owner[t]];
      src = br.src;
      len = br.len;
      dst = br.dst;
      const int32_t q0 = (static_cast<int32_t>(t) - br.base) * kCopyUnit;
      const int32_t q1 = q0 + kCopyUnit < len ? q0 + kCopyUnit : len;
      a = q0 == 0 ? 0 : next_run_start(ind_old + src, q0, len, sh, &bad);
      b = q1 == len ? len : next_run_start(ind_old + src, q1, len, sh, &bad);
    } else {
      const int64_t l = t - units;
      const int32_t r = l < rows1 ? lists[list_stride + l] : lists[l - rows1];
      src = src_new[r];
      dst = ptr_new[r];
      len = ptr_new[r + 1] - dst;
      a = 0;
      b = len;
    }
    const int32_t *ind = ind_old + src;
    const float *val = val_old ? val_old + src : nullptr;
    int32_t *kout = ind_new + dst;
    float *vout = val_new ? val_new + dst : nullptr;
    int32_t s = a;
    while (s < b) {
      const int32_t i = s + lane;
      const bool in = i < b;
      const int32_t c = in ? ind[i] : 0;
      const int32_t cn = in && i + 1 < len ? ind[i + 1] : 0x7fffffff;
      if (in && cn <= c) bad = true;
      // Lane i ends a run when the next entry is past the task or in another
      // block.
      const uint64_t me = ballot(in && (i + 1 == b || (cn >> sh) != (c >> sh)));
      if (me == 0) {
        // The run at s is longer than the window.
        s = place_long_run(rb, ind, val, delta, s, b, len, sh, kout, vout, &bad);
        continue;
      }
      // Whole runs in lanes [0, last].
      const int last = 63 - __builtin_clzll(me);
      const bool mine = lane <= last;
      int32_t key = mine ? c + delta[c] : 0x7fffffff;
      float v = (mine && val) ? val[i] : 0.0f;
      // Run of this lane: [rs, re] in lanes.
      const uint64_t starts = (me << 1) | 1ull;
      const int rs = 63 - __builtin_clzll(starts & (~0ull >> (63 - lane)));
      const int re = __builtin_ctzll(me & (~0ull << lane) | (1ull << 63));
      const uint32_t span = mine ? static_cast<uint32_t>(re - rs + 1) : 1u;
      const uint32_t longest = wave_max_u32(span);
      int pos = lane;
      if (longest > static_cast<uint32_t>(kRunRankCap)) {
        // Sort the whole-run prefix (lanes past `last` hold the padding key).
        group_sort<kWave>(key, v, lane);
      } else if (longest > 1) {
        int rank = 0;
        for (int d = 1; d < static_cast<int>(longest); ++d) {
          const int32_t up = __shfl(key, lane - d >= 0 ? lane - d : 0, kWave);
          const int32_t dn = __shfl(key, lane + d < kWave ? lane + d : kWave - 1, kWave);
          rank += (lane - d >= rs && up < key) ? 1 : 0;
          rank += (lane + d <= re && dn < key) ? 1 : 0;
        }
        pos = rs + rank;
      }
      if (mine) {
        kout[s + pos] = key;
        if (vout) vout[s + pos] = v;
      }
      s += last + 1;
    }
  }
  if (ballot(bad) != 0 && lane == 0) atomicOr(&ctl->unsorted, 1);
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
void launch_permute_g(Context &ctx, int32_t n, const int32_t *src_new, const int32_t *ind_old,
                      const float *val_old, const int32_t *col_map, const int16_t *delta,
                      const int32_t *ptr_new, int32_t *ind_new, float *val_new,
                      int32_t *key_tmp, float *val_tmp, int32_t *lists, int32_t list_stride,
                      Ctl *ctl, BigRow *big_rows, int32_t *big_owner, bool allow_runs) {
  constexpr int U = G <= 16 ? 4 : 2;
  constexpr int rows_per_block = 4 * (kWave / G) * U;
  const int g = ctx.grid_for(ceil_div64(n, rows_per_block), 256, 4);
  permute_rows<G, U><<<g, 256, 0, ctx.stream>>>(n, src_new, ind_old, val_old, col_map, delta,
                                                ptr_new, ind_new, val_new, key_tmp, val_tmp,
                                                lists, list_stride, ctl, big_rows, big_owner,
                                                allow_runs ? 1 : 0);
  SP_LAUNCH_CHECK();
}

void launch_permute(Context &ctx, int G, int32_t n, const int32_t *src_new,
                    const int32_t *ind_old, const float *val_old, const int32_t *col_map,
                    const int16_t *delta, const int32_t *ptr_new, int32_t *ind_new,
                    float *val_new, int32_t *key_tmp, float *val_tmp, int32_t *lists,
                    int32_t list_stride, Ctl *ctl, BigRow *big_rows, int32_t *big_owner,
                    bool allow_runs) {
  switch (G) {
#define SP_CASE(V)                                                                       \
  case V:                                                                                \
    launch_permute_g<V>(ctx, n, src_new, ind_old, val_old, col_map, delta, ptr_new,      \
                        ind_new, val_new, key_tmp, val_tmp, lists, list_stride, ctl,     \
                        big_rows, big_owner, allow_runs);                                \
    break;
    SP_CASE(4) SP_CASE(8) SP_CASE(16) SP_CASE(32) SP_CASE(64)
#undef SP_CASE
  default:
    SP_EXPECT(false, "internal: bad group width");
  }
}

// Copies the units of the big rows permute_rows registered (the host knows
// their count from the control words).
void launch_copy_big(Context &ctx, int32_t units, const int32_t *ind_old, const float *val_old,
                     const int32_t *col_map, const BigRow *big_rows, const int32_t *big_owner,
                     int32_t *ind_out, float *val_out) {
  if (units <= 0) return;
  const int gb = ctx.grid_for(units, 256, 4);
  copy_big_rows<<<gb, 256, 0, ctx.stream>>>(ind_old, val_old, col_map, units, big_rows,
                                            big_owner, ind_out, val_out);
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
                ws_bytes<Ctl>(1) + ws_bytes<BigRow>(static_cast<size_t>(max_big_rows(nnz))) +
                ws_bytes<int32_t>(static_cast<size_t>(max_copy_units(nnz))) + ws_bytes<int32_t>(n);
  const int64_t scan_tiles = ceil_div64(static_cast<int64_t>(n) + 1, kScanTileElems);
  if (symmetric) {
    need += ws_bytes<int32_t>(n) + ws_bytes<int16_t>(n) + ws_bytes<int32_t>(nnz) +
            ws_bytes<float>(nnz) + ws_bytes<int32_t>(3 * (static_cast<size_t>(n) + 2));
  }
  ctx.reserve(need);
  int32_t *scan_tmp = ctx.take<int32_t>(scan_tmp_elems(static_cast<int64_t>(n) + 1));
  Ctl *ctl = ctx.take<Ctl>(1);
  BigRow *big_rows = ctx.take<BigRow>(static_cast<size_t>(max_big_rows(nnz)));
  int32_t *big_owner = ctx.take<int32_t>(static_cast<size_t>(max_copy_units(nnz)));
  int32_t *src_new = ctx.take<int32_t>(n);
  int32_t *old2new = symmetric ? ctx.take<int32_t>(n) : nullptr;

  const int row_grid = ctx.grid_for(ceil_div64(n, 256), 256, 4);

  prepare_rows<<<dim3(static_cast<unsigned>(scan_tiles)), kPrepBlock, 0, ctx.stream>>>(
      n, d_ptr_old, d_new_order, d_ptr_new, src_new, old2new, scan_tmp, ctl);
  SP_LAUNCH_CHECK();
  scan_i32_from_totals(ctx, d_ptr_new, d_ptr_new, static_cast<int64_t>(n) + 1, true, scan_tmp);

  // Lanes per row: the average row length rounded up to a power of two,
  // between 4 and 64.
  int G = 4;
  while (G < 64 && static_cast<int64_t>(G) * n < nnz) G <<= 1;

  // The control words come back once, after the copy kernel; the stages after
  // it are launched only when they have rows.
  Ctl hc{};
  auto read_ctl = [&] {
    SP_HIP(hipMemcpyAsync(ctx.host_words, ctl, sizeof(Ctl), hipMemcpyDeviceToHost, ctx.stream));
    ctx.sync();
    std::memcpy(&hc, ctx.host_words, sizeof(Ctl));
  };

  if (!symmetric) {
    launch_permute(ctx, G, n, src_new, d_ind_old, d_val_old, nullptr, nullptr, d_ptr_new,
                   d_ind_new, d_val_new, nullptr, nullptr, nullptr, 0, ctl, big_rows,
                   big_owner, false);
    read_ctl();
    if (hc.big.units > 0) {
      launch_copy_big(ctx, hc.big.units, d_ind_old, d_val_old, nullptr, big_rows, big_owner,
                      d_ind_new, d_val_new);
      ctx.sync();
    }
    return;
  }

  int16_t *delta = ctx.take<int16_t>(n);
  int32_t *unsorted = ctx.take<int32_t>(nnz);
  float *val_unsorted = ctx.take<float>(nnz);
  // Row lists of the three sort stages, one array with stride n + 2.
  const int32_t stride = n + 2;
  int32_t *lists = ctx.take<int32_t>(3 * static_cast<size_t>(stride));
  int32_t *list1 = lists, *long_rows = lists + stride, *huge_rows = lists + 2 * stride;
  const float *vo = with_vals ? d_val_old : nullptr;
  float *vn = with_vals ? d_val_new : nullptr;
  float *vt = with_vals ? val_unsorted : nullptr;

  narrow_map<<<std::min(row_grid, 4 * ctx.num_cus), 256, 0, ctx.stream>>>(n, old2new, delta,
                                                                          ctl);
  SP_LAUNCH_CHECK();
  // Rows of at most 2G entries are remapped, sorted and written in one pass;
  // longer rows are listed by length for the stage that sorts them, and the
  // stages launch only when their lists have rows.
  launch_permute(ctx, G, n, src_new, d_ind_old, vo, old2new, delta, d_ptr_new, d_ind_new, vn,
                 unsorted, vt, lists, stride, ctl, big_rows, big_owner, true);
  read_ctl();
  // Run mode, as permute_rows decided it from the same control words: every
  // listed row is gathered and sorted run by run in one launch.  A row that
  // is not strictly increasing sends the call's long rows back through the
  // full sorts below, after a second permute_rows pass without run mode.
  if (hc.wide == 0 && hc.sh <= kRunMaxBits) {
    const int64_t tasks = static_cast<int64_t>(hc.big.units) + hc.counts[0] + hc.counts[1];
    if (tasks == 0) return;
    const int g = std::min<int>(ctx.grid_for(ceil_div64(tasks, kRunWaves), kRunBlock, 8),
                                8 * ctx.num_cus);
    sort_runs<<<g, kRunBlock, 0, ctx.stream>>>(lists, stride, hc.counts[0], hc.counts[1],
                                               hc.big.units, d_ptr_new, src_new, big_rows,
                                               big_owner, d_ind_old, vo, delta, hc.sh,
                                               d_ind_new, vn, ctl);
    SP_LAUNCH_CHECK();
    read_ctl();
    if (hc.unsorted == 0) return;
    fill_u32(ctx, ctl, kCtlListWords, 0u);
    launch_permute(ctx, G, n, src_new, d_ind_old, vo, old2new, delta, d_ptr_new, d_ind_new,
                   vn, unsorted, vt, lists, stride, ctl, big_rows, big_owner, false);
    read_ctl();
  }
  const bool narrow = hc.wide == 0;
  bool queued = false;
  if (hc.counts[0] > 0) {
    const int g = std::min<int>(ctx.grid_for(ceil_div64(hc.counts[0], 4), 256, 4),
                                4 * ctx.num_cus);
    sort_rows_wave<<<g, 256, 0, ctx.stream>>>(list1, hc.counts[0], d_ptr_new, unsorted, vt,
                                              d_ind_new, vn);
    SP_LAUNCH_CHECK();
    queued = true;
  }
  if (hc.counts[1] > 0) {
    sort_rows_block<<<std::min(hc.counts[1], ctx.num_cus * 4), kBlockSortThreads, 0,
                      ctx.stream>>>(d_ptr_new, long_rows, hc.counts[1], src_new, d_ind_old, vo,
                                    old2new, delta, narrow, d_ind_new, vn);
    SP_LAUNCH_CHECK();
    queued = true;
  }
  if (hc.counts[2] > 0) {
    // Rows past kBlockSortCap: copied unsorted (their units registered by
    // permute_rows), then one device-wide sort.
    launch_copy_big(ctx, hc.big.units, d_ind_old, vo, old2new, big_rows, big_owner, unsorted,
                    vt);
    sort_huge_rows(ctx, n, d_ptr_new, huge_rows, hc.counts[2], unsorted, vt, d_ind_new, vn,
                   list1, scan_tmp);
    queued = true;
  }
  if (queued) ctx.sync();
}
