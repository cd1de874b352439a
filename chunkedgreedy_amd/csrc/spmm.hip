// spmm.hip -- CSR SpMM (fp32, row-major dense operands) and the SpMM
// benchmark hook.
//
// C = A * B with A in CSR (n x n, values), B and C dense n x N, row-major.
// The reference times cuSPARSE CSR ALG1 behind sporder_bench_cusparse_spmm
// (sporder/src/bench_cusparse_spmm.cu:25-103) and its harness calls
// SpMMMethod.run (bench/spmm/spmm_bench/base.py:48-59) on row-major B from
// torch.randn.  These kernels replace both.
//
// Row-split: a group of G lanes owns one row, each lane 4 adjacent columns
// (float4), so a wave covers 64/G rows and one B row gather per nonzero is a
// single coalesced G*16-byte access.  The row's (col, val) pairs are loaded
// cooperatively by the group and broadcast by lane shuffles, U B-rows in
// flight per group.  Stated accumulation order (bit-identical to the CPU loop
// of oracle_spmm_csr):
//   - a row with at most kLongRow nonzeros: acc = fmaf(a_p, B[col_p][j], acc)
//     over p in CSR order starting at 0.0f;
//   - a longer row: split into segments of kSegLen nonzeros from the row's
//     start; each segment is such a chain from 0.0f, and
//     C[i][j] = ((P_0 + P_1) + P_2) + ... left to right.
// The segments of long rows are processed by many row groups of a second
// launch (so one hub row does not serialise the whole SpMM), and a third
// launch adds each long row's partials in the stated order.  For N <= 32
// (8 or more rows per wave) the row groups of a wave claim its 64 rows
// dynamically, so short rows do not wait for a long neighbour.
//
// Merge-path: the nonzeros are cut into equal spans per wave (a row longer
// than a span is split); each span's partial row sums are added into C with
// atomics after the short rows are written directly.  The result equals the
// row-split one up to the rounding of the split rows.
#include "common.hpp"
#include "philox.hpp"

#include <mutex>

namespace sporder_hip {

namespace {

constexpr int kSpmmBlock = 256;
constexpr int kSpmmWaves = kSpmmBlock / kWave;
constexpr int kSpmmDepth = 8; // B rows in flight per row group
constexpr int kLongRow = SPORDER_SPMM_LONG_ROW;
constexpr int kSegLen = SPORDER_SPMM_SEGMENT;
constexpr int kTileRows = kSpmmTileRows; // rows of a tile of an SpMM plan

// Long rows: rows past kLongRow nonzeros leave the row-split launch, which
// appends a descriptor; each becomes nseg segment units whose partials the
// fixup launch adds.
struct LongRow {
  int32_t row;
  int32_t base; // first unit (also its first partial row)
  int32_t nseg;
  int32_t pad;
};
struct LongCtl {
  int32_t rows;     // long rows registered
  int32_t segments; // units allocated
};

// Registers a row of `len` > kLongRow nonzeros (one lane per row).
__device__ __forceinline__ void register_row(LongCtl *ctl, LongRow *longs, int32_t *owner,
                                             int32_t row, int32_t len) {
  const int32_t nseg = (len + kSegLen - 1) / kSegLen;
  const int32_t id = atomicAdd(&ctl->rows, 1);
  const int32_t base = atomicAdd(&ctl->segments, nseg);
  longs[id] = LongRow{row, base, nseg, 0};
  for (int32_t q = 0; q < nseg; ++q) owner[base + q] = id;
}

__device__ __forceinline__ float4 scale4(float d, float4 v) {
  return make_float4(d * v.x, d * v.y, d * v.z, d * v.w);
}

// The row scale applied to a finished row (rs null: none), rounded once per
// element: the value an elementwise product of the result would hold.
__device__ __forceinline__ float4 row_scaled(const float *__restrict__ rs, int64_t row, float4 v) {
  return rs != nullptr ? scale4(rs[row], v) : v;
}

// A[s, e) x B on the group's float4 column slice col0 (col_ok false: lanes
// past N).  Every lane of the wave calls it together; groups with different
// ranges iterate until the longest is done.  Accumulates fmaf in CSR order
// starting from 0.0f.  With CS the B row gathered for nonzero p is first
// multiplied by cs[p] (the scale of that nonzero's column, streamed beside
// the values), cs[p] * B[col][j] rounded once: the value an elementwise
// product of B by a column-scale vector would hold.
template <int G, bool CS>
__device__ __forceinline__ float4 group_dot(int32_t s, int32_t e, const int32_t *__restrict__ ind,
                                            const float *__restrict__ val, int32_t N,
                                            int32_t col0, bool col_ok,
                                            const float *__restrict__ B, int gl, int gbase,
                                            const float *__restrict__ cs) {
  constexpr int U = kSpmmDepth;
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int32_t pb = s;; pb += G) {
    const int32_t rem = e - pb;
    if (ballot(rem > 0) == 0) break;
    int32_t my_c = 0;
    float my_v = 0.0f, my_d = 1.0f;
    if (gl < rem) {
      my_c = __builtin_nontemporal_load(ind + pb + gl);
      my_v = __builtin_nontemporal_load(val + pb + gl);
      if constexpr (CS) my_d = __builtin_nontemporal_load(cs + pb + gl);
    }
    const int32_t cnt = rem < G ? rem : G;
    // Wave maximum of cnt bounds the broadcast loop.
    const int32_t cmax = static_cast<int32_t>(
        wave_max_u32(static_cast<uint32_t>(cnt > 0 ? cnt : 0)));
    for (int32_t t = 0; t < cmax; t += U) {
      int32_t c[U];
      float v[U], d[U];
      float4 b[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        c[u] = __shfl(my_c, gbase + ((t + u) & (G - 1)), kWave);
        v[u] = __shfl(my_v, gbase + ((t + u) & (G - 1)), kWave);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (t + u < cnt && col_ok) {
          b[u] = *reinterpret_cast<const float4 *>(B + static_cast<int64_t>(c[u]) * N + col0);
        }
      }
      // Each lane loaded its own nonzero's column scale; it is shared out only
      // after the B rows are requested, so the gathers do not wait for it.
      if constexpr (CS) {
#pragma unroll
        for (int u = 0; u < U; ++u) d[u] = __shfl(my_d, gbase + ((t + u) & (G - 1)), kWave);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (t + u < cnt && col_ok) {
          if constexpr (CS) b[u] = scale4(d[u], b[u]);
          acc.x = fmaf(v[u], b[u].x, acc.x);
          acc.y = fmaf(v[u], b[u].y, acc.y);
          acc.z = fmaf(v[u], b[u].z, acc.z);
          acc.w = fmaf(v[u], b[u].w, acc.w);
        }
      }
    }
  }
  return acc;
}

__device__ __forceinline__ void store_nt(float *dst, float4 v) {
  __builtin_nontemporal_store(v.x, dst + 0);
  __builtin_nontemporal_store(v.y, dst + 1);
  __builtin_nontemporal_store(v.z, dst + 2);
  __builtin_nontemporal_store(v.w, dst + 3);
}

// One pass over the rows, 64/G rows per wave, one wave per row set (no grid
// stride).  Rows longer than kLongRow are registered in `longs` for the
// segment launch (when `longs` is null every row is done here, in one chain).
// C is written with non-temporal stores: it is not read again by this launch
// and would only evict B from the caches.  rs / cs (CS): the row scales and
// the per-nonzero column scales of a scaled product (null rs: none).
template <int G, bool CS>
__global__ void __launch_bounds__(kSpmmBlock)
    spmm_rowsplit_v4(int32_t n, const int32_t *__restrict__ ptr,
                     const int32_t *__restrict__ ind,
                     const float *__restrict__ val, int32_t N,
                     const float *__restrict__ B, float *__restrict__ C,
                     LongCtl *ctl, LongRow *longs, int32_t *owner,
                     const int32_t *__restrict__ tiles, int64_t ntiles,
                     const float *__restrict__ rs, const float *__restrict__ cs) {
  constexpr int kRowsPerWave = kWave / G;
  const int lane = lane_id();
  const int sub = lane / G;  // row slot within the wave
  const int gl = lane % G;   // lane within the row group
  const int gbase = sub * G; // first lane of the group
  // Each tile of kTileRows consecutive rows on one XCD (rows in a good order
  // share B rows in that L2), tiles dealt to the XCDs in turn (an index-ordered
  // skew, hubs first, is spread over all of them).  Measured against one
  // contiguous eighth of the rows per XCD, outputs identical: C5 in degree
  // order N = 128 8.17 -> 3.87 ms, C3 reordered N = 256 22.9 -> 19.5 ms,
  // RGG20 -5 %, C4 -4 %, C2 and C2r in planted order unchanged (a round-robin
  // of single workgroups instead took C2r from 0.56 to 0.74 ms).
  constexpr int64_t kTileWgs = kTileRows / (kRowsPerWave * kSpmmWaves) > 0
                                   ? kTileRows / (kRowsPerWave * kSpmmWaves) : 1;
  const int64_t wave = xcd_tile_block(kTileWgs) * kSpmmWaves + threadIdx.x / kWave;
  // With a tile list, G waves cover each listed tile of kTileRows rows; the
  // waves past the list (the grid is whole blocks) take no row.
  const int64_t row = tiles == nullptr ? wave * kRowsPerWave + sub
                      : wave / G < ntiles
                          ? static_cast<int64_t>(tiles[wave / G]) * kTileRows +
                                (wave % G) * kRowsPerWave + sub
                          : static_cast<int64_t>(n);
  const bool row_ok = row < n;
  int32_t s = row_ok ? ptr[row] : 0;
  const int32_t e = row_ok ? ptr[row + 1] : 0;
  const bool is_long = longs != nullptr && e - s > kLongRow;
  if (is_long) {
    if (gl == 0) register_row(ctl, longs, owner, static_cast<int32_t>(row), e - s);
    s = e; // the segment launch computes this row
  }
  for (int32_t col0 = gl * 4; col0 - gl * 4 < N; col0 += G * 4) {
    const bool col_ok = col0 < N;
    const float4 acc = group_dot<G, CS>(s, e, ind, val, N, col0, col_ok, B, gl, gbase, cs);
    if (row_ok && col_ok && !is_long) store_nt(C + row * N + col0, row_scaled(rs, row, acc));
  }
}

// Dynamic row-split for N <= 32 (one float4 column pass): a wave owns 64
// consecutive rows and its 64/G row groups claim them in order, a group taking
// the next unclaimed row as soon as its current one ends, so groups of one wave
// do not wait for the longest row among them.  Each row is still one group's
// fmaf chain in CSR order.  Row bounds come from one coalesced load of the
// wave's 65 row pointers; rows longer than kLongRow are registered for the
// segment launch as in spmm_rowsplit_v4.
template <int G, bool CS>
__global__ void __launch_bounds__(kSpmmBlock)
    spmm_rows_dyn(int32_t n, const int32_t *__restrict__ ptr, const int32_t *__restrict__ ind,
                  const float *__restrict__ val, int32_t N, const float *__restrict__ B,
                  float *__restrict__ C, LongCtl *ctl, LongRow *longs, int32_t *owner,
                  const int32_t *__restrict__ tiles, int64_t ntiles,
                  const float *__restrict__ rs, const float *__restrict__ cs) {
  static_assert(kTileRows == kWave, "a wave owns one tile");
  constexpr int U = kSpmmDepth;
  constexpr int RPW = kWave / G;
  const int lane = lane_id();
  const int sub = lane / G, gl = lane % G, gbase = sub * G;
  // A workgroup's 4 waves own 4 * 64 consecutive rows (one XCD); workgroups
  // are dealt to the XCDs in turn, as the hardware dispatches them.
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * kSpmmWaves + threadIdx.x / kWave;
  if (tiles != nullptr && wave >= ntiles) return; // past the list (whole blocks)
  const int64_t r0 = tiles == nullptr ? wave * kWave : static_cast<int64_t>(tiles[wave]) * kWave;
  if (r0 >= n) return;
  const int32_t nrows = static_cast<int32_t>(n - r0 < kWave ? n - r0 : kWave);
  // Lane i holds ptr[r0 + i] (i <= nrows); ptr[r0 + 64] separately.
  const int32_t pl = ptr[r0 + (lane < nrows ? lane : nrows)];
  const int32_t p_last = ptr[r0 + nrows];
  const int col0 = gl * 4;
  const bool col_ok = col0 < N;

  int32_t row = sub < nrows ? sub : -1; // local row of this group, -1 idle
  int32_t next = RPW;                   // wave-uniform: next unclaimed local row
  int32_t p = 0, e = 0;
  bool is_long = false;
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  // A claimed row longer than kLongRow goes to the segment launch and counts
  // as finished at once.
  auto take_long = [&]() {
    if (longs != nullptr && row >= 0 && e - p > kLongRow) {
      if (gl == 0) register_row(ctl, longs, owner, static_cast<int32_t>(r0 + row), e - p);
      is_long = true;
      p = e;
    }
  };
  // Every lane takes part in each shuffle (a source lane that is inactive for
  // a ds_bpermute reads as 0); the selects come after.
  {
    const int32_t a = __shfl(pl, row >= 0 ? row : 0, kWave);
    const int32_t bi = row >= 0 ? row + 1 : 0;
    const int32_t bs = __shfl(pl, bi < kWave ? bi : kWave - 1, kWave);
    p = row >= 0 ? a : 0;
    e = row >= 0 ? (bi < kWave ? bs : p_last) : 0;
    take_long();
  }
  while (true) {
    // Retire finished rows and claim new ones until every group has work or
    // the wave's rows are used up.
    while (true) {
      const bool fin = row >= 0 && p >= e;
      if (fin && !is_long && col_ok) {
        store_nt(C + (r0 + row) * N + col0, row_scaled(rs, r0 + row, acc));
      }
      const uint64_t fmask = ballot(fin && gl == 0);
      if (fmask == 0) break;
      const int32_t rank = __popcll(fmask & ((1ull << gbase) - 1ull));
      const int32_t cand = next + rank;
      const int32_t ci = cand < nrows ? cand : 0;
      const int32_t a = __shfl(pl, ci, kWave);
      const int32_t bi = ci + 1;
      const int32_t bs = __shfl(pl, bi < kWave ? bi : kWave - 1, kWave);
      const int32_t b = bi < kWave ? bs : p_last;
      if (fin) {
        row = cand < nrows ? cand : -1;
        p = row >= 0 ? a : 0;
        e = row >= 0 ? b : 0;
        is_long = false;
        acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        take_long();
      }
      next += __popcll(fmask);
    }
    if (ballot(row >= 0) == 0) break;
    // One step: up to G nonzeros per group, U B rows in flight.
    const int32_t rem = row >= 0 ? e - p : 0;
    int32_t my_c = 0;
    float my_v = 0.0f, my_d = 1.0f;
    if (gl < rem) {
      my_c = __builtin_nontemporal_load(ind + p + gl);
      my_v = __builtin_nontemporal_load(val + p + gl);
      if constexpr (CS) my_d = __builtin_nontemporal_load(cs + p + gl);
    }
    const int32_t cnt = rem < G ? rem : G;
    const int32_t cmax = static_cast<int32_t>(wave_max_u32(static_cast<uint32_t>(cnt)));
    for (int32_t t = 0; t < cmax; t += U) {
      int32_t c[U];
      float v[U], d[U];
      float4 bv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        c[u] = __shfl(my_c, gbase + ((t + u) & (G - 1)), kWave);
        v[u] = __shfl(my_v, gbase + ((t + u) & (G - 1)), kWave);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (t + u < cnt && col_ok) {
          bv[u] = *reinterpret_cast<const float4 *>(B + static_cast<int64_t>(c[u]) * N + col0);
        }
      }
      if constexpr (CS) {
#pragma unroll
        for (int u = 0; u < U; ++u) d[u] = __shfl(my_d, gbase + ((t + u) & (G - 1)), kWave);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (t + u < cnt && col_ok) {
          if constexpr (CS) bv[u] = scale4(d[u], bv[u]);
          acc.x = fmaf(v[u], bv[u].x, acc.x);
          acc.y = fmaf(v[u], bv[u].y, acc.y);
          acc.z = fmaf(v[u], bv[u].z, acc.z);
          acc.w = fmaf(v[u], bv[u].w, acc.w);
        }
      }
    }
    if (row >= 0) p += cnt;
  }
}

// Segment units of the long rows: each row group computes one segment's
// partial into `part` (unit-major, N floats per unit).  Grid-stride over the
// units registered by the row-split launch.  The partials are added by the
// next launch: handing them over inside this one would need a device-scope
// release/acquire per unit, which on MI355X writes back and invalidates the
// XCD's L2 and so evicts every other wave's B rows.
template <int G, bool CS>
__global__ void __launch_bounds__(kSpmmBlock)
    spmm_long_segments(const int32_t *__restrict__ ptr, const int32_t *__restrict__ ind,
                       const float *__restrict__ val, int32_t N,
                       const float *__restrict__ B, const LongCtl *__restrict__ ctl,
                       const LongRow *__restrict__ longs, const int32_t *__restrict__ owner,
                       float *__restrict__ part, const float *__restrict__ cs) {
  constexpr int kRowsPerWave = kWave / G;
  const int lane = lane_id();
  const int sub = lane / G, gl = lane % G, gbase = sub * G;
  const int64_t wave0 = static_cast<int64_t>(blockIdx.x) * kSpmmWaves + threadIdx.x / kWave;
  const int64_t nwaves = static_cast<int64_t>(gridDim.x) * kSpmmWaves;
  const int32_t units = ctl->segments;
  for (int64_t ub = wave0 * kRowsPerWave; ub < units; ub += nwaves * kRowsPerWave) {
    const int64_t u = ub + sub;
    const bool ok = u < units;
    int32_t s = 0, e = 0;
    if (ok) {
      const LongRow lr = longs[owner[u]];
      const int32_t rs = ptr[lr.row], re = ptr[lr.row + 1];
      s = rs + static_cast<int32_t>(u - lr.base) * kSegLen;
      e = s + kSegLen < re ? s + kSegLen : re;
    }
    for (int32_t col0 = gl * 4; col0 - gl * 4 < N; col0 += G * 4) {
      const bool col_ok = col0 < N;
      const float4 acc = group_dot<G, CS>(s, e, ind, val, N, col0, col_ok, B, gl, gbase, cs);
      if (ok && col_ok) *reinterpret_cast<float4 *>(part + u * N + col0) = acc;
    }
  }
}

// C[row] = ((P_0 + P_1) + P_2) + ... for each long row, one row group per row,
// eight partial rows in flight; then the row scale (rs null: none).
template <int G>
__global__ void __launch_bounds__(kSpmmBlock)
    spmm_long_fixup(int32_t N, float *__restrict__ C, const LongCtl *__restrict__ ctl,
                    const LongRow *__restrict__ longs, const float *__restrict__ part,
                    const float *__restrict__ rs) {
  constexpr int kRowsPerWave = kWave / G;
  const int lane = lane_id();
  const int sub = lane / G, gl = lane % G;
  const int64_t wave0 = static_cast<int64_t>(blockIdx.x) * kSpmmWaves + threadIdx.x / kWave;
  const int64_t nwaves = static_cast<int64_t>(gridDim.x) * kSpmmWaves;
  const int32_t rows = ctl->rows;
  for (int64_t t = wave0 * kRowsPerWave + sub; t < rows; t += nwaves * kRowsPerWave) {
    const LongRow lr = longs[t];
    const float *p0 = part + static_cast<int64_t>(lr.base) * N;
    for (int32_t col0 = gl * 4; col0 < N; col0 += G * 4) {
      float4 sum = *reinterpret_cast<const float4 *>(p0 + col0);
      int32_t q = 1;
      for (; q + 8 <= lr.nseg; q += 8) {
        float4 v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          v[i] = *reinterpret_cast<const float4 *>(p0 + static_cast<int64_t>(q + i) * N + col0);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          sum.x = sum.x + v[i].x;
          sum.y = sum.y + v[i].y;
          sum.z = sum.z + v[i].z;
          sum.w = sum.w + v[i].w;
        }
      }
      for (; q < lr.nseg; ++q) {
        const float4 v = *reinterpret_cast<const float4 *>(p0 + static_cast<int64_t>(q) * N + col0);
        sum.x = sum.x + v.x;
        sum.y = sum.y + v.y;
        sum.z = sum.z + v.z;
        sum.w = sum.w + v.w;
      }
      store_nt(C + static_cast<int64_t>(lr.row) * N + col0, row_scaled(rs, lr.row, sum));
    }
  }
}

// Scalar fallback for widths that are not a multiple of 4 (or unaligned
// operands): one wave per row, lanes over columns, same stated order (long
// rows as segment chains added left to right).
__global__ void __launch_bounds__(kSpmmBlock)
    spmm_rowsplit_scalar(int32_t n, const int32_t *__restrict__ ptr,
                         const int32_t *__restrict__ ind,
                         const float *__restrict__ val, int32_t N,
                         const float *__restrict__ B, float *__restrict__ C,
                         const float *__restrict__ rs = nullptr,
                         const float *__restrict__ cs = nullptr) {
  const int lane = lane_id();
  const int64_t wave0 =
      (blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x) / kWave;
  const int64_t nwaves = static_cast<int64_t>(gridDim.x) * blockDim.x / kWave;
  for (int64_t row = wave0; row < n; row += nwaves) {
    const int32_t s = ptr[row], e = ptr[row + 1];
    const int32_t seg = e - s > kLongRow ? kSegLen : (e - s > 0 ? e - s : 1);
    for (int32_t j = lane; j < N; j += kWave) {
      float sum = 0.0f;
      for (int32_t q0 = s; q0 < e || q0 == s; q0 += seg) {
        const int32_t q1 = q0 + seg < e ? q0 + seg : e;
        float acc = 0.0f;
        for (int32_t p = q0; p < q1; ++p) {
          const float b = B[static_cast<int64_t>(ind[p]) * N + j];
          acc = fmaf(val[p], cs != nullptr ? cs[p] * b : b, acc);
        }
        sum = (q0 == s) ? acc : sum + acc;
      }
      C[row * N + j] = rs != nullptr ? rs[row] * sum : sum;
    }
  }
}

// ---- merge-path ---------------------------------------------------------------

// Each wave owns nonzeros [w*span, (w+1)*span).  Rows entirely inside the span
// are written with a plain store; the partial sums of rows cut by a span edge
// are added with atomics into C, which the caller zeroes for those rows first.
__global__ void __launch_bounds__(kSpmmBlock)
    spmm_merge_path(int32_t n, int32_t nnz, const int32_t *__restrict__ ptr,
                    const int32_t *__restrict__ ind,
                    const float *__restrict__ val, int32_t N,
                    const float *__restrict__ B, float *__restrict__ C,
                    int32_t span) {
  const int lane = lane_id();
  const int64_t wave =
      (blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x) / kWave;
  const int64_t p0 = wave * span;
  if (p0 >= nnz) return;
  const int32_t p_begin = static_cast<int32_t>(p0);
  const int32_t p_end = static_cast<int32_t>(p0 + span > nnz ? nnz : p0 + span);
  // First row whose end passes p_begin: largest r with ptr[r] <= p_begin.
  int32_t lo = 0, hi = n - 1;
  while (lo < hi) {
    int32_t mid = lo + (hi - lo + 1) / 2;
    if (ptr[mid] <= p_begin) {
      lo = mid;
    } else {
      hi = mid - 1;
    }
  }
  int32_t row = lo;
  int32_t p = p_begin;
  while (p < p_end) {
    while (ptr[row + 1] <= p) ++row; // skip empty rows
    const int32_t rs = ptr[row], re = ptr[row + 1];
    const int32_t seg_end = re < p_end ? re : p_end;
    const bool whole = rs >= p_begin && re <= p_end;
    for (int32_t j = lane; j < N; j += kWave) {
      float acc = 0.0f;
      for (int32_t q = p; q < seg_end; ++q) {
        acc = fmaf(val[q], B[static_cast<int64_t>(ind[q]) * N + j], acc);
      }
      if (whole) {
        C[static_cast<int64_t>(row) * N + j] = acc;
      } else {
        atomicAdd(&C[static_cast<int64_t>(row) * N + j], acc);
      }
    }
    p = seg_end;
  }
}

// Merge-path on row groups: group g (G lanes, one float4 column slice each)
// owns the nonzeros [g*span, (g+1)*span) and walks the pieces of the rows
// they cover, in row order, with the pipelined gathers of the row-split
// kernels.  A row lying wholly inside the span is stored; the piece of a row
// cut by a span edge is added into C with float atomics (those rows are
// zeroed first), so a cut row's value depends on the order of the atomics:
// within 1e-5 of the row-split result, not bit-identical.  Row ends come from
// a window of G row pointers held in the group's lanes; empty rows are
// skipped (the prepare launch zeroes them).  N > 4G is covered by repeating
// the walk per column slice.
template <int G>
__global__ void __launch_bounds__(kSpmmBlock)
    spmm_merge_v4(int32_t n, int32_t nnz, const int32_t *__restrict__ ptr,
                  const int32_t *__restrict__ ind, const float *__restrict__ val, int32_t N,
                  const float *__restrict__ B, float *__restrict__ C, int32_t span,
                  const int32_t *__restrict__ start_row) {
  constexpr int U = kSpmmDepth;
  constexpr uint64_t kGroupMask = G == kWave ? ~0ull : ((1ull << G) - 1ull);
  const int lane = lane_id();
  const int sub = lane / G, gl = lane % G, gbase = sub * G;
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * kSpmmWaves + threadIdx.x / kWave;
  const int64_t grp = wave * (kWave / G) + sub;
  const int64_t p0_64 = grp * static_cast<int64_t>(span);
  const bool has = p0_64 < nnz;
  const int32_t p0 = has ? static_cast<int32_t>(p0_64) : nnz;
  const int32_t p1 =
      has ? static_cast<int32_t>(p0_64 + span < nnz ? p0_64 + span : nnz) : nnz;
  // First row of the span: the row holding nonzero p0 (from the prepare launch).
  const int32_t first = has ? start_row[grp] : -1;
  for (int32_t cb = 0; cb < N; cb += 4 * G) {
    const int32_t col0 = cb + gl * 4;
    const bool col_ok = col0 < N;
    int32_t row = first;
    int32_t wbase = first >= 0 ? first : 0;
    int32_t win = ptr[wbase + 1 + gl < n ? wbase + 1 + gl : n]; // ptr[wbase + 1 + gl]
    const int32_t w0 = __shfl(win, gbase, kWave);               // every lane shuffles
    int32_t rs = row >= 0 ? ptr[row] : 0;
    int32_t re = row >= 0 ? w0 : 0;
    int32_t p = row >= 0 ? (rs > p0 ? rs : p0) : 0;
    int32_t e = row >= 0 ? (re < p1 ? re : p1) : 0;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    while (true) {
      // Retire finished pieces and move each such group to its span's next
      // row, until every group has work or is done.
      while (true) {
        const bool fin = row >= 0 && p >= e;
        if (fin && col_ok) {
          float *dst = C + static_cast<int64_t>(row) * N + col0;
          if (rs >= p0 && re <= p1) {
            store_nt(dst, acc);
          } else {
            atomicAdd(dst + 0, acc.x);
            atomicAdd(dst + 1, acc.y);
            atomicAdd(dst + 2, acc.z);
            atomicAdd(dst + 3, acc.w);
          }
        }
        if (ballot(fin) == 0) break;
        // Next row of the span with nonzeros: the first row after `row` whose
        // end passes re (empty rows in between were zeroed by the prepare
        // launch).  The window moves on while it holds only empty rows; the
        // span's nonzeros past re guarantee such a row before n.
        bool seek = fin && re < p1;
        int32_t after = row; // rows up to `after` are done
        int32_t next = -1, nend = 0;
        while (ballot(seek) != 0) {
          if (seek && after + 1 - wbase >= G) {
            wbase = after + 1;
            win = ptr[wbase + 1 + gl < n ? wbase + 1 + gl : n];
          }
          const bool c = seek && gl >= after + 1 - wbase && win > re;
          const uint64_t gm = (ballot(c) >> gbase) & kGroupMask;
          const int32_t off = gm != 0 ? static_cast<int32_t>(__builtin_ctzll(gm)) : 0;
          const int32_t wend = __shfl(win, gbase + off, kWave);
          if (seek) {
            if (gm != 0) {
              next = wbase + off;
              nend = wend;
              seek = false;
            } else {
              after = wbase + G - 1;
            }
          }
        }
        if (fin) {
          if (next >= 0) {
            rs = re; // empty rows in between start and end there too
            re = nend;
            row = next;
            p = rs;
            e = re < p1 ? re : p1;
            acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
          } else {
            row = -1;
          }
        }
      }
      if (ballot(row >= 0) == 0) break;
      // One step: up to G nonzeros per group, U B rows in flight.
      const int32_t rem = row >= 0 ? e - p : 0;
      int32_t my_c = 0;
      float my_v = 0.0f;
      if (gl < rem) {
        my_c = __builtin_nontemporal_load(ind + p + gl);
        my_v = __builtin_nontemporal_load(val + p + gl);
      }
      const int32_t cnt = rem < G ? rem : G;
      const int32_t cmax = static_cast<int32_t>(wave_max_u32(static_cast<uint32_t>(cnt)));
      for (int32_t t = 0; t < cmax; t += U) {
        int32_t c[U];
        float v[U];
        float4 bv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          c[u] = __shfl(my_c, gbase + ((t + u) & (G - 1)), kWave);
          v[u] = __shfl(my_v, gbase + ((t + u) & (G - 1)), kWave);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (t + u < cnt && col_ok) {
            bv[u] = *reinterpret_cast<const float4 *>(B + static_cast<int64_t>(c[u]) * N + col0);
          }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (t + u < cnt && col_ok) {
            acc.x = fmaf(v[u], bv[u].x, acc.x);
            acc.y = fmaf(v[u], bv[u].y, acc.y);
            acc.z = fmaf(v[u], bv[u].z, acc.z);
            acc.w = fmaf(v[u], bv[u].w, acc.w);
          }
        }
      }
      if (row >= 0) p += cnt;
    }
  }
}

// Zero C rows that the merge-path kernel will accumulate into (rows crossing
// a span boundary) and rows with no nonzeros (no span writes them).  With
// start_row, also record for every span the row holding its first nonzero.
// One lane per row for the bounds, the wave for each row it zeroes.
__global__ void spmm_merge_prepare(int32_t n, const int32_t *__restrict__ ptr,
                                   int32_t N, float *__restrict__ C, int32_t span,
                                   int32_t *__restrict__ start_row) {
  const int lane = lane_id();
  const int64_t wave0 =
      (blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x) / kWave;
  const int64_t nwaves = static_cast<int64_t>(gridDim.x) * blockDim.x / kWave;
  for (int64_t rb = wave0 * kWave; rb < n; rb += nwaves * kWave) {
    const int64_t r = rb + lane;
    int32_t rs = 0, re = 0;
    if (r < n) {
      rs = ptr[r];
      re = ptr[r + 1];
    }
    const bool empty = r < n && rs == re;
    const bool split = r < n && !empty && (rs / span) != ((re - 1) / span);
    if (start_row != nullptr && r < n && !empty) {
      for (int64_t sp = (static_cast<int64_t>(rs) + span - 1) / span; sp * span < re; ++sp) {
        start_row[sp] = static_cast<int32_t>(r);
      }
    }
    uint64_t m = ballot(empty || split);
    while (m) {
      const int64_t row = rb + __builtin_ctzll(m);
      m &= m - 1;
      for (int32_t j = lane; j < N; j += kWave) C[row * N + j] = 0.0f;
    }
  }
}

// vals[i] = U(0,1] from counter (i/4, stream) under key = seed.
__global__ void fill_uniform(int64_t count, float *__restrict__ vals, uint64_t seed,
                             uint32_t stream_id) {
  for (int64_t q = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
       q * 4 < count; q += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    uint4 r = philox4x32_10(
        make_uint4(static_cast<uint32_t>(q), static_cast<uint32_t>(q >> 32), stream_id, 0u),
        make_uint2(static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32)));
    uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      int64_t i = q * 4 + u;
      if (i < count) vals[i] = static_cast<float>((w[u] >> 8) + 1u) * (1.0f / 16777216.0f);
    }
  }
}

// Workspace of the long-row segments for an n x n CSR with nnz nonzeros and
// N columns: descriptors, unit owners and unit partials, sized for the most
// long rows and segments nnz nonzeros allow.
// Scales of a scaled product diag(row) A diag(col) B: `row` holds n row
// scales, `col` nnz per-nonzero column scales (col[p] = the scale of column
// ind[p]); null: no scale on that side.
struct SpmmScale {
  const float *row = nullptr;
  const float *col = nullptr;
};

struct SpmmLongWs {
  LongCtl *ctl;
  LongRow *longs;
  int32_t *owner;
  float *part;
};

int64_t max_long_rows(int32_t nnz) { return nnz / (kLongRow + 1) + 1; }
int64_t max_segments(int32_t nnz) { return nnz / kSegLen + max_long_rows(nnz) + 1; }

SpmmLongWs take_long_ws(Context &ctx, int32_t nnz, int32_t N) {
  SpmmLongWs w;
  w.ctl = ctx.take<LongCtl>(1);
  w.longs = ctx.take<LongRow>(static_cast<size_t>(max_long_rows(nnz)));
  w.owner = ctx.take<int32_t>(static_cast<size_t>(max_segments(nnz)));
  w.part = ctx.take<float>(static_cast<size_t>(max_segments(nnz)) * N);
  return w;
}

template <int G, bool CS>
void launch_rowsplit_gs(Context &ctx, int32_t n, int32_t nnz, const int32_t *ptr,
                        const int32_t *ind, const float *val, int32_t N, const float *B,
                        float *C, const SpmmLongWs &w, int64_t seg_cap, int64_t long_cap,
                        const int32_t *tiles, int64_t ntiles, const float *rs,
                        const float *cs) {
  constexpr int rpw = kWave / G;
  // Without a long-row workspace (a plan found no row past kLongRow) the row
  // launch computes every row and the segment launches are not made.
  const bool long_rows = w.ctl != nullptr;
  if (long_rows) fill_u32(ctx, w.ctl, sizeof(LongCtl) / 4, 0u);
  // Narrow widths (G <= 8 lanes per row, 8+ rows per wave) lose most to
  // row-length imbalance inside a wave: claim rows dynamically there.  With
  // wider rows the fixed assignment keeps more waves in flight.  With a tile
  // list only the listed tiles' rows are computed.
  const int64_t waves = tiles == nullptr ? ceil_div64(n, rpw) : ntiles * (kTileRows / rpw);
  if (G <= 8 && N <= 4 * G) {
    const int64_t dyn_waves = tiles == nullptr ? ceil_div64(n, kWave) : ntiles;
    const int64_t blocks = ceil_div64(dyn_waves, kSpmmWaves);
    spmm_rows_dyn<G, CS><<<dim3(static_cast<unsigned>(blocks)), kSpmmBlock, 0, ctx.stream>>>(
        n, ptr, ind, val, N, B, C, w.ctl, w.longs, w.owner, tiles, ntiles, rs, cs);
  } else {
    const int64_t blocks = ceil_div64(waves, kSpmmWaves);
    spmm_rowsplit_v4<G, CS><<<dim3(static_cast<unsigned>(blocks)), kSpmmBlock, 0,
                              ctx.stream>>>(n, ptr, ind, val, N, B, C, w.ctl, w.longs,
                                            w.owner, tiles, ntiles, rs, cs);
  }
  SP_LAUNCH_CHECK();
  if (!long_rows) return;
  // Persistent grid over the registered segment units (none: exits at once).
  const int g = ctx.grid_for(ceil_div64(seg_cap, rpw * kSpmmWaves), kSpmmBlock, 2);
  spmm_long_segments<G, CS><<<g, kSpmmBlock, 0, ctx.stream>>>(ptr, ind, val, N, B, w.ctl,
                                                                w.longs, w.owner, w.part, cs);
  SP_LAUNCH_CHECK();
  const int gf = ctx.grid_for(ceil_div64(long_cap, rpw * kSpmmWaves), kSpmmBlock, 2);
  spmm_long_fixup<G><<<gf, kSpmmBlock, 0, ctx.stream>>>(N, C, w.ctl, w.longs, w.part, rs);
  SP_LAUNCH_CHECK();
}

template <int G>
void launch_rowsplit_g(Context &ctx, int32_t n, int32_t nnz, const int32_t *ptr,
                       const int32_t *ind, const float *val, int32_t N, const float *B,
                       float *C, const SpmmLongWs &w, int64_t seg_cap, int64_t long_cap,
                       const int32_t *tiles, int64_t ntiles, const SpmmScale &sc) {
  if (sc.col != nullptr) {
    launch_rowsplit_gs<G, true>(ctx, n, nnz, ptr, ind, val, N, B, C, w, seg_cap, long_cap,
                                tiles, ntiles, sc.row, sc.col);
  } else {
    launch_rowsplit_gs<G, false>(ctx, n, nnz, ptr, ind, val, N, B, C, w, seg_cap, long_cap,
                                 tiles, ntiles, sc.row, nullptr);
  }
}

} // namespace

size_t spmm_ws_bytes(int32_t nnz, int32_t N) {
  return ws_bytes<LongCtl>(1) + ws_bytes<LongRow>(static_cast<size_t>(max_long_rows(nnz))) +
         ws_bytes<int32_t>(static_cast<size_t>(max_segments(nnz))) +
         ws_bytes<float>(static_cast<size_t>(max_segments(nnz)) * N);
}

// Row-split SpMM in the stated order.  `w` holds room for `long_cap` long rows
// and `seg_cap` segments (take_long_ws: the most nnz nonzeros allow).  `sc`:
// the scales of a scaled product (SpmmScale; null: none).
void spmm_rowsplit(Context &ctx, int32_t n, int32_t nnz, const int32_t *ptr,
                   const int32_t *ind, const float *val, int32_t N, const float *B, float *C,
                   const SpmmLongWs &w, int64_t seg_cap = -1, int64_t long_cap = -1,
                   const int32_t *tiles = nullptr, int64_t ntiles = 0,
                   const SpmmScale &sc = SpmmScale{}) {
  if (seg_cap < 0) seg_cap = max_segments(nnz);
  if (long_cap < 0) long_cap = max_long_rows(nnz);
  bool aligned = (N % 4 == 0) && (reinterpret_cast<uintptr_t>(B) % 16 == 0) &&
                 (reinterpret_cast<uintptr_t>(C) % 16 == 0);
  if (!aligned) {
    SP_EXPECT(tiles == nullptr, "internal: tile lists need aligned float4 operands");
    int g = ctx.grid_for(ceil_div64(n, kSpmmBlock / kWave), kSpmmBlock, 8);
    spmm_rowsplit_scalar<<<g, kSpmmBlock, 0, ctx.stream>>>(n, ptr, ind, val, N, B, C, sc.row,
                                                           sc.col);
    SP_LAUNCH_CHECK();
    return;
  }
  int32_t q = N / 4; // float4 columns
  if (q <= 1) {
    launch_rowsplit_g<1>(ctx, n, nnz, ptr, ind, val, N, B, C, w, seg_cap, long_cap,
                          tiles, ntiles, sc);
  } else if (q <= 2) {
    launch_rowsplit_g<2>(ctx, n, nnz, ptr, ind, val, N, B, C, w, seg_cap, long_cap,
                          tiles, ntiles, sc);
  } else if (q <= 4) {
    launch_rowsplit_g<4>(ctx, n, nnz, ptr, ind, val, N, B, C, w, seg_cap, long_cap,
                          tiles, ntiles, sc);
  } else if (q <= 8) {
    launch_rowsplit_g<8>(ctx, n, nnz, ptr, ind, val, N, B, C, w, seg_cap, long_cap,
                          tiles, ntiles, sc);
  } else if (q <= 16) {
    launch_rowsplit_g<16>(ctx, n, nnz, ptr, ind, val, N, B, C, w, seg_cap, long_cap,
                          tiles, ntiles, sc);
  } else if (q <= 32) {
    launch_rowsplit_g<32>(ctx, n, nnz, ptr, ind, val, N, B, C, w, seg_cap, long_cap,
                          tiles, ntiles, sc);
  } else {
    launch_rowsplit_g<64>(ctx, n, nnz, ptr, ind, val, N, B, C, w, seg_cap, long_cap,
                          tiles, ntiles, sc);
  }
}

void spmm_rowsplit_tiles(Context &ctx, int32_t n, int32_t nnz, const int32_t *ptr,
                         const int32_t *ind, const float *val, int32_t N, const float *B,
                         float *C, const int32_t *tiles, int64_t ntiles, bool long_rows) {
  SpmmLongWs w{nullptr, nullptr, nullptr, nullptr};
  if (long_rows) {
    ctx.reserve(spmm_ws_bytes(nnz, N));
    w = take_long_ws(ctx, nnz, N);
  }
  spmm_rowsplit(ctx, n, nnz, ptr, ind, val, N, B, C, w, -1, -1, tiles, ntiles);
}

template <int G>
void launch_merge_g(Context &ctx, int32_t n, int32_t nnz, const int32_t *ptr,
                    const int32_t *ind, const float *val, int32_t N, const float *B, float *C) {
  constexpr int gpw = kWave / G; // row groups per wave
  // Span: about two groups per resident group slot, at least G * kSpmmDepth
  // nonzeros (one full gather pipeline per group).
  const int64_t groups = static_cast<int64_t>(ctx.num_cus) *
                         (ctx.max_threads_per_cu / kWave) * gpw * 2;
  int64_t span64 = ceil_div64(nnz > 0 ? nnz : 1, groups);
  if (span64 < G * kSpmmDepth) span64 = G * kSpmmDepth;
  const int32_t span = static_cast<int32_t>(span64);
  const int64_t spans = ceil_div64(nnz, span);
  ctx.reserve(ws_bytes<int32_t>(static_cast<size_t>(spans) + 1));
  int32_t *start_row = ctx.take<int32_t>(static_cast<size_t>(spans) + 1);
  const int gp = ctx.grid_for(ceil_div64(n, kSpmmBlock), kSpmmBlock, 4);
  spmm_merge_prepare<<<gp, kSpmmBlock, 0, ctx.stream>>>(n, ptr, N, C, span, start_row);
  SP_LAUNCH_CHECK();
  if (nnz == 0) return;
  const int64_t blocks = ceil_div64(spans, gpw * kSpmmWaves);
  spmm_merge_v4<G><<<dim3(static_cast<unsigned>(blocks)), kSpmmBlock, 0, ctx.stream>>>(
      n, nnz, ptr, ind, val, N, B, C, span, start_row);
  SP_LAUNCH_CHECK();
}

void spmm_merge(Context &ctx, int32_t n, int32_t nnz, const int32_t *ptr,
                const int32_t *ind, const float *val, int32_t N, const float *B,
                float *C) {
  const bool aligned = (N % 4 == 0) && (reinterpret_cast<uintptr_t>(B) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(C) % 16 == 0);
  if (aligned) {
    const int32_t q = N / 4; // float4 columns
    if (q <= 1) {
      launch_merge_g<1>(ctx, n, nnz, ptr, ind, val, N, B, C);
    } else if (q <= 2) {
      launch_merge_g<2>(ctx, n, nnz, ptr, ind, val, N, B, C);
    } else if (q <= 4) {
      launch_merge_g<4>(ctx, n, nnz, ptr, ind, val, N, B, C);
    } else if (q <= 8) {
      launch_merge_g<8>(ctx, n, nnz, ptr, ind, val, N, B, C);
    } else if (q <= 16) {
      launch_merge_g<16>(ctx, n, nnz, ptr, ind, val, N, B, C);
    } else if (q <= 32) {
      launch_merge_g<32>(ctx, n, nnz, ptr, ind, val, N, B, C);
    } else {
      launch_merge_g<64>(ctx, n, nnz, ptr, ind, val, N, B, C);
    }
    return;
  }
  // Widths that are not a multiple of 4 (or unaligned operands): one wave per
  // span, lanes over columns.
  int64_t slots = static_cast<int64_t>(ctx.num_cus) * (ctx.max_threads_per_cu / kWave) * 2;
  int64_t span64 = ceil_div64(nnz > 0 ? nnz : 1, slots);
  if (span64 < 32) span64 = 32;
  int32_t span = static_cast<int32_t>(span64);
  int gp = ctx.grid_for(ceil_div64(n, kSpmmBlock), kSpmmBlock, 4);
  spmm_merge_prepare<<<gp, kSpmmBlock, 0, ctx.stream>>>(n, ptr, N, C, span, nullptr);
  SP_LAUNCH_CHECK();
  if (nnz == 0) return;
  int64_t waves = ceil_div64(nnz, span);
  int64_t blocks = ceil_div64(waves, kSpmmBlock / kWave);
  spmm_merge_path<<<dim3(static_cast<unsigned>(blocks)), kSpmmBlock, 0, ctx.stream>>>(
      n, nnz, ptr, ind, val, N, B, C, span);
  SP_LAUNCH_CHECK();
}

// ---- no-allocation variant -----------------------------------------------------
//
// sporder_spmm_csr_noalloc runs the row-split kernels above with their scratch
// (long-row descriptors, segment owners, segment partial rows) carved from
// `scratch`, a file-scope device array of SPORDER_SPMM_NOALLOC_SCRATCH_BYTES
// that every GPU the library runs on holds until the process ends.  Host code
// never passes the array's name to a kernel (in host code it is a host-side
// stand-in, not a device address): each device's address comes from
// hipGetSymbolAddress, taken once per device when a context is created on it
// (spmm_noalloc_setup) and kept in noalloc_ptr.  Every call on one GPU uses
// that GPU's array, so calls that overlap on one GPU (two contexts, two
// threads) race; the counters it holds are cleared by a fill kernel at the
// start of each call.

namespace {

constexpr size_t kNoAllocBytes = SPORDER_SPMM_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

constexpr int kMaxDevices = 64;
std::mutex noalloc_mu;
void *noalloc_ptr[kMaxDevices] = {};
// Held by a no-allocation call from its first use of the device's array to
// its final synchronize, so that calls of this process on one device run one
// after another (other processes hold arrays of their own).
std::mutex noalloc_call_mu[kMaxDevices];

// Rows past kLongRow nonzeros and their segments: ctl->rows, ctl->segments
// (zeroed by the caller).  Grid-stride, one lane per row.
__global__ void __launch_bounds__(256)
    spmm_count_long(int32_t n, const int32_t *__restrict__ ptr, LongCtl *ctl) {
  int32_t rows = 0, segs = 0;
  for (int64_t r = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; r < n;
       r += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int32_t len = ptr[r + 1] - ptr[r];
    if (len > kLongRow) {
      rows += 1;
      segs += (len + kSegLen - 1) / kSegLen;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    rows += __shfl_xor(rows, off, kWave);
    segs += __shfl_xor(segs, off, kWave);
  }
  if (lane_id() == 0 && rows != 0) {
    atomicAdd(&ctl->rows, rows);
    atomicAdd(&ctl->segments, segs);
  }
}

} // namespace

// Takes this device's address of `scratch` (the device must be current).
void spmm_noalloc_setup(int device) {
  SP_EXPECT(device >= 0 && device < kMaxDevices, "device index out of range");
  std::lock_guard<std::mutex> lock(noalloc_mu);
  if (noalloc_ptr[device] != nullptr) return;
  void *p = nullptr;
  SP_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
  SP_EXPECT(p != nullptr, "hipGetSymbolAddress returned no address for the SpMM scratch");
  noalloc_ptr[device] = p;
}

namespace {

void *noalloc_scratch(int device) {
  std::lock_guard<std::mutex> lock(noalloc_mu);
  void *p = device >= 0 && device < kMaxDevices ? noalloc_ptr[device] : nullptr;
  SP_EXPECT(p != nullptr, "no SpMM scratch address for this device (context not set up)");
  return p;
}

} // namespace

} // namespace sporder_hip

using namespace sporder_hip;

extern "C" {

int32_t sporder_spmm_csr_noalloc(sporder_context_t h, int32_t n, int32_t nnz,
                                 const int32_t *d_ptr, const int32_t *d_ind,
                                 const float *d_val, int32_t cols, const float *d_b,
                                 float *d_c) {
  SP_EXPECT(h != nullptr, "null context");
  SP_EXPECT(n >= 1 && nnz >= 0, "expect n >= 1 and nnz >= 0");
  SP_EXPECT(cols >= 1, "cols must be >= 1");
  Context &ctx = h->impl;
  char *base = static_cast<char *>(noalloc_scratch(ctx.device));
  std::lock_guard<std::mutex> call_lock(noalloc_call_mu[ctx.device]);
  const bool aligned = (cols % 4 == 0) && (reinterpret_cast<uintptr_t>(d_b) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(d_c) % 16 == 0);
  if (!aligned) {
    // One wave per row in the stated order: no scratch.
    int g = ctx.grid_for(ceil_div64(n, kSpmmBlock / kWave), kSpmmBlock, 8);
    spmm_rowsplit_scalar<<<g, kSpmmBlock, 0, ctx.stream>>>(n, d_ptr, d_ind, d_val, cols, d_b,
                                                           d_c);
    SP_LAUNCH_CHECK();
    ctx.sync();
    return 0;
  }
  // Exact need: count the long rows and their segments first.
  LongCtl *ctl = reinterpret_cast<LongCtl *>(base);
  fill_u32(ctx, ctl, sizeof(LongCtl) / 4, 0u);
  const int gc = ctx.grid_for(ceil_div64(n, 256), 256, 2);
  spmm_count_long<<<gc, 256, 0, ctx.stream>>>(n, d_ptr, ctl);
  SP_LAUNCH_CHECK();
  SP_HIP(hipMemcpyAsync(ctx.host_words, ctl, sizeof(LongCtl), hipMemcpyDeviceToHost,
                        ctx.stream));
  ctx.sync();
  const int64_t long_rows = ctx.host_words[0], segments = ctx.host_words[1];
  const size_t need = ws_bytes<LongCtl>(1) + ws_bytes<LongRow>(static_cast<size_t>(long_rows)) +
                      ws_bytes<int32_t>(static_cast<size_t>(segments)) +
                      ws_bytes<float>(static_cast<size_t>(segments) * cols);
  if (need > kNoAllocBytes) return SPORDER_SPMM_NOALLOC_TOO_LARGE;
  SpmmLongWs w;
  size_t off = ws_bytes<LongCtl>(1);
  w.ctl = ctl;
  w.longs = reinterpret_cast<LongRow *>(base + off);
  off += ws_bytes<LongRow>(static_cast<size_t>(long_rows));
  w.owner = reinterpret_cast<int32_t *>(base + off);
  off += ws_bytes<int32_t>(static_cast<size_t>(segments));
  w.part = reinterpret_cast<float *>(base + off);
  spmm_rowsplit(ctx, n, nnz, d_ptr, d_ind, d_val, cols, d_b, d_c, w, segments, long_rows);
  ctx.sync();
  return 0;
}

void sporder_spmm_csr(sporder_context_t h, int32_t n, int32_t nnz,
                      const int32_t *d_ptr, const int32_t *d_ind, const float *d_val,
                      int32_t cols, const float *d_b, float *d_c,
                      sporder_spmm_algo_t algo, float *kernel_ms) {
  SP_EXPECT(h != nullptr, "null context");
  SP_EXPECT(n >= 1 && nnz >= 0, "expect n >= 1 and nnz >= 0");
  SP_EXPECT(cols >= 1, "cols must be >= 1");
  SP_EXPECT(algo == SPORDER_SPMM_AUTO || algo == SPORDER_SPMM_ROW_SPLIT ||
                algo == SPORDER_SPMM_MERGE_PATH,
            "invalid SpMM algorithm");
  Context &ctx = h->impl;
  EventSpan t;
  t.create(kernel_ms != nullptr);
  if (algo != SPORDER_SPMM_MERGE_PATH) ctx.reserve(spmm_ws_bytes(nnz, cols));
  t.begin(ctx.stream);
  if (algo == SPORDER_SPMM_MERGE_PATH) {
    spmm_merge(ctx, n, nnz, d_ptr, d_ind, d_val, cols, d_b, d_c);
  } else {
    const SpmmLongWs w = take_long_ws(ctx, nnz, cols);
    spmm_rowsplit(ctx, n, nnz, d_ptr, d_ind, d_val, cols, d_b, d_c, w);
  }
  t.end(ctx.stream);
  ctx.sync();
  if (kernel_ms) *kernel_ms = t.ms();
  t.destroy();
}

void sporder_spmm_csr_scaled(sporder_context_t h, int32_t n, int32_t nnz,
                             const int32_t *d_ptr, const int32_t *d_ind, const float *d_val,
                             int32_t cols, const float *d_b, const float *d_row_scale,
                             const float *d_nz_col_scale, float *d_c, float *kernel_ms) {
  SP_EXPECT(h != nullptr, "null context");
  SP_EXPECT(n >= 1 && nnz >= 0, "expect n >= 1 and nnz >= 0");
  SP_EXPECT(cols >= 1, "cols must be >= 1");
  Context &ctx = h->impl;
  EventSpan t;
  t.create(kernel_ms != nullptr);
  ctx.reserve(spmm_ws_bytes(nnz, cols));
  t.begin(ctx.stream);
  const SpmmLongWs w = take_long_ws(ctx, nnz, cols);
  SpmmScale sc;
  sc.row = d_row_scale;
  sc.col = d_nz_col_scale;
  spmm_rowsplit(ctx, n, nnz, d_ptr, d_ind, d_val, cols, d_b, d_c, w, -1, -1, nullptr, 0, sc);
  t.end(ctx.stream);
  ctx.sync();
  if (kernel_ms) *kernel_ms = t.ms();
  t.destroy();
}

void sporder_bench_cusparse_spmm(sporder_context_t h, int32_t n, int32_t nnz,
                                 const int32_t *d_ptr, const int32_t *d_ind,
                                 int32_t cols, int32_t warmup, int32_t repeat,
                                 uint64_t seed, float *wall_ms) {
  // Argument checks: reference sporder/src/sporder.cpp:172-173.
  SP_EXPECT(h != nullptr, "null context");
  SP_EXPECT(warmup >= 0 && repeat >= 0, "warmup and repeat must be >= 0");
  SP_EXPECT(cols >= 1, "cols must be >= 1");
  SP_EXPECT(n >= 1 && nnz >= 0, "expect n >= 1 and nnz >= 0");
  Context &ctx = h->impl;
  const int64_t b_count = static_cast<int64_t>(n) * cols;
  ctx.reserve(ws_bytes<float>(nnz) + 2 * ws_bytes<float>(b_count) + spmm_ws_bytes(nnz, cols));
  float *a_val = ctx.take<float>(nnz);
  float *b = ctx.take<float>(b_count);
  float *c = ctx.take<float>(b_count);
  const SpmmLongWs w = take_long_ws(ctx, nnz, cols);
  // Values from seed ^ 0xA and seed ^ 0xB, as the reference keys its two fills
  // (bench_cusparse_spmm.cu:40,44).
  int ga = ctx.grid_for(ceil_div64(ceil_div64(nnz, 4), 256), 256, 4);
  fill_uniform<<<ga, 256, 0, ctx.stream>>>(nnz, a_val, seed ^ 0xAull, 0u);
  SP_LAUNCH_CHECK();
  int gb = ctx.grid_for(ceil_div64(ceil_div64(b_count, 4), 256), 256, 4);
  fill_uniform<<<gb, 256, 0, ctx.stream>>>(b_count, b, seed ^ 0xBull, 1u);
  SP_LAUNCH_CHECK();
  for (int32_t i = 0; i < warmup; ++i) {
    spmm_rowsplit(ctx, n, nnz, d_ptr, d_ind, a_val, cols, b, c, w);
  }
  ctx.sync();
  EventSpan t;
  t.create(true);
  t.begin(ctx.stream);
  for (int32_t i = 0; i < repeat; ++i) {
    spmm_rowsplit(ctx, n, nnz, d_ptr, d_ind, a_val, cols, b, c, w);
  }
  t.end(ctx.stream);
  ctx.sync();
  *wall_ms = repeat > 0 ? t.ms() / repeat : 0.0f;
  t.destroy();
}

} // extern "C"
