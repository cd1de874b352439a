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
// cooperatively by the group and broadcast by lane shuffles.  Every output
// element is acc = fmaf(a_p, B[col_p][j], acc) over p in CSR order starting
// at 0.0f, bit-identical to a sequential CPU loop.
//
// Merge-path: the nonzeros are cut into equal spans per wave (a row longer
// than a span is split); each span's partial row sums are added into C with
// atomics after the short rows are written directly.  The result equals the
// row-split one up to the rounding of the split rows.
#include "common.hpp"

namespace sporder_hip {

namespace {

constexpr int kSpmmBlock = 256;

template <int G>
__global__ void __launch_bounds__(kSpmmBlock)
    spmm_rowsplit_v4(int32_t n, const int32_t *__restrict__ ptr,
                     const int32_t *__restrict__ ind,
                     const float *__restrict__ val, int32_t N,
                     const float *__restrict__ B, float *__restrict__ C) {
  constexpr int kRowsPerWave = kWave / G;
  const int lane = lane_id();
  const int sub = lane / G;  // row slot within the wave
  const int gl = lane % G;   // lane within the row group
  const int gbase = sub * G; // first lane of the group
  const int64_t wave0 =
      (blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x) / kWave;
  const int64_t nwaves = static_cast<int64_t>(gridDim.x) * blockDim.x / kWave;

  for (int64_t rb = wave0 * kRowsPerWave; rb < n; rb += nwaves * kRowsPerWave) {
    const int64_t row = rb + sub;
    const bool row_ok = row < n;
    const int32_t s = row_ok ? ptr[row] : 0;
    const int32_t e = row_ok ? ptr[row + 1] : 0;
    for (int32_t col0 = gl * 4; col0 - gl * 4 < N; col0 += G * 4) {
      const bool col_ok = col0 < N;
      float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      for (int32_t pb = s;; pb += G) {
        // Wave-uniform loop: continue while any group has nonzeros left.
        int32_t rem = e - pb;
        if (ballot(rem > 0) == 0) break;
        int32_t my_c = 0;
        float my_v = 0.0f;
        if (gl < rem) {
          my_c = ind[pb + gl];
          my_v = val[pb + gl];
        }
        int32_t cnt = rem < G ? rem : G;
        // Wave max of cnt bounds the broadcast loop.
        int32_t cmax = cnt;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
          int32_t o = __shfl_xor(cmax, off, kWave);
          cmax = o > cmax ? o : cmax;
        }
        for (int32_t t = 0; t < cmax; t += 4) {
          int32_t c[4];
          float v[4];
          float4 b[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            c[u] = __shfl(my_c, gbase + ((t + u) & (G - 1)), kWave);
            v[u] = __shfl(my_v, gbase + ((t + u) & (G - 1)), kWave);
          }
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            if (t + u < cnt && col_ok) {
              b[u] = *reinterpret_cast<const float4 *>(
                  B + static_cast<int64_t>(c[u]) * N + col0);
            }
          }
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            if (t + u < cnt && col_ok) {
              acc.x = fmaf(v[u], b[u].x, acc.x);
              acc.y = fmaf(v[u], b[u].y, acc.y);
              acc.z = fmaf(v[u], b[u].z, acc.z);
              acc.w = fmaf(v[u], b[u].w, acc.w);
            }
          }
        }
      }
      if (row_ok && col_ok) {
        *reinterpret_cast<float4 *>(C + row * N + col0) = acc;
      }
    }
  }
}

// Scalar fallback for widths that are not a multiple of 4: one wave per row,
// lanes over columns.
__global__ void __launch_bounds__(kSpmmBlock)
    spmm_rowsplit_scalar(int32_t n, const int32_t *__restrict__ ptr,
                         const int32_t *__restrict__ ind,
                         const float *__restrict__ val, int32_t N,
                         const float *__restrict__ B, float *__restrict__ C) {
  const int lane = lane_id();
  const int64_t wave0 =
      (blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x) / kWave;
  const int64_t nwaves = static_cast<int64_t>(gridDim.x) * blockDim.x / kWave;
  for (int64_t row = wave0; row < n; row += nwaves) {
    const int32_t s = ptr[row], e = ptr[row + 1];
    for (int32_t j = lane; j < N; j += kWave) {
      float acc = 0.0f;
      for (int32_t p = s; p < e; ++p) {
        acc = fmaf(val[p], B[static_cast<int64_t>(ind[p]) * N + j], acc);
      }
      C[row * N + j] = acc;
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

// Zero C rows that the merge-path kernel will accumulate into (rows crossing
// a span boundary) and rows with no nonzeros (no span writes them).
__global__ void spmm_merge_prepare(int32_t n, const int32_t *__restrict__ ptr,
                                   int32_t N, float *__restrict__ C, int32_t span) {
  const int lane = lane_id();
  const int64_t wave0 =
      (blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x) / kWave;
  const int64_t nwaves = static_cast<int64_t>(gridDim.x) * blockDim.x / kWave;
  for (int64_t row = wave0; row < n; row += nwaves) {
    const int32_t rs = ptr[row], re = ptr[row + 1];
    const bool empty = rs == re;
    const bool split = !empty && (rs / span) != ((re - 1) / span);
    if (empty || split) {
      for (int32_t j = lane; j < N; j += kWave) C[row * N + j] = 0.0f;
    }
  }
}

// ---- Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11) -------------------------

__device__ __forceinline__ uint4 philox4x32_10(uint4 ctr, uint2 key) {
  const uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u;
  const uint32_t W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    uint32_t hi0 = __umulhi(M0, ctr.x), lo0 = M0 * ctr.x;
    uint32_t hi1 = __umulhi(M1, ctr.z), lo1 = M1 * ctr.z;
    ctr = make_uint4(hi1 ^ ctr.y ^ key.x, lo1, hi0 ^ ctr.w ^ key.y, lo0);
    key.x += W0;
    key.y += W1;
  }
  return ctr;
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

template <int G>
void launch_rowsplit_g(Context &ctx, int32_t n, const int32_t *ptr, const int32_t *ind,
                       const float *val, int32_t N, const float *B, float *C) {
  constexpr int rpw = kWave / G;
  int64_t waves = ceil_div64(n, rpw);
  int g = ctx.grid_for(ceil_div64(waves, kSpmmBlock / kWave), kSpmmBlock, 8);
  spmm_rowsplit_v4<G><<<g, kSpmmBlock, 0, ctx.stream>>>(n, ptr, ind, val, N, B, C);
  SP_LAUNCH_CHECK();
}

} // namespace

void spmm_rowsplit(Context &ctx, int32_t n, const int32_t *ptr, const int32_t *ind,
                   const float *val, int32_t N, const float *B, float *C) {
  bool aligned = (N % 4 == 0) && (reinterpret_cast<uintptr_t>(B) % 16 == 0) &&
                 (reinterpret_cast<uintptr_t>(C) % 16 == 0);
  if (!aligned) {
    int g = ctx.grid_for(ceil_div64(n, kSpmmBlock / kWave), kSpmmBlock, 8);
    spmm_rowsplit_scalar<<<g, kSpmmBlock, 0, ctx.stream>>>(n, ptr, ind, val, N, B, C);
    SP_LAUNCH_CHECK();
    return;
  }
  int32_t q = N / 4; // float4 columns
  if (q <= 1) {
    launch_rowsplit_g<1>(ctx, n, ptr, ind, val, N, B, C);
  } else if (q <= 2) {
    launch_rowsplit_g<2>(ctx, n, ptr, ind, val, N, B, C);
  } else if (q <= 4) {
    launch_rowsplit_g<4>(ctx, n, ptr, ind, val, N, B, C);
  } else if (q <= 8) {
    launch_rowsplit_g<8>(ctx, n, ptr, ind, val, N, B, C);
  } else if (q <= 16) {
    launch_rowsplit_g<16>(ctx, n, ptr, ind, val, N, B, C);
  } else if (q <= 32) {
    launch_rowsplit_g<32>(ctx, n, ptr, ind, val, N, B, C);
  } else {
    launch_rowsplit_g<64>(ctx, n, ptr, ind, val, N, B, C);
  }
}

void spmm_merge(Context &ctx, int32_t n, int32_t nnz, const int32_t *ptr,
                const int32_t *ind, const float *val, int32_t N, const float *B,
                float *C) {
  // Span: about 2 waves per CU slot of work, at least 32 nonzeros.
  int64_t slots = static_cast<int64_t>(ctx.num_cus) * (ctx.max_threads_per_cu / kWave) * 2;
  int64_t span64 = ceil_div64(nnz > 0 ? nnz : 1, slots);
  if (span64 < 32) span64 = 32;
  int32_t span = static_cast<int32_t>(span64);
  int gp = ctx.grid_for(ceil_div64(n, kSpmmBlock / kWave), kSpmmBlock, 4);
  spmm_merge_prepare<<<gp, kSpmmBlock, 0, ctx.stream>>>(n, ptr, N, C, span);
  SP_LAUNCH_CHECK();
  if (nnz == 0) return;
  int64_t waves = ceil_div64(nnz, span);
  int64_t blocks = ceil_div64(waves, kSpmmBlock / kWave);
  spmm_merge_path<<<dim3(static_cast<unsigned>(blocks)), kSpmmBlock, 0, ctx.stream>>>(
      n, nnz, ptr, ind, val, N, B, C, span);
  SP_LAUNCH_CHECK();
}

} // namespace sporder_hip

using namespace sporder_hip;

extern "C" {

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
  t.begin(ctx.stream);
  if (algo == SPORDER_SPMM_MERGE_PATH) {
    spmm_merge(ctx, n, nnz, d_ptr, d_ind, d_val, cols, d_b, d_c);
  } else {
    spmm_rowsplit(ctx, n, d_ptr, d_ind, d_val, cols, d_b, d_c);
  }
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
  ctx.reserve(ws_bytes<float>(nnz) + 2 * ws_bytes<float>(b_count));
  float *a_val = ctx.take<float>(nnz);
  float *b = ctx.take<float>(b_count);
  float *c = ctx.take<float>(b_count);
  // Values from seed ^ 0xA and seed ^ 0xB, as the reference keys its two fills
  // (bench_cusparse_spmm.cu:40,44).
  int ga = ctx.grid_for(ceil_div64(ceil_div64(nnz, 4), 256), 256, 4);
  fill_uniform<<<ga, 256, 0, ctx.stream>>>(nnz, a_val, seed ^ 0xAull, 0u);
  SP_LAUNCH_CHECK();
  int gb = ctx.grid_for(ceil_div64(ceil_div64(b_count, 4), 256), 256, 4);
  fill_uniform<<<gb, 256, 0, ctx.stream>>>(b_count, b, seed ^ 0xBull, 1u);
  SP_LAUNCH_CHECK();
  for (int32_t i = 0; i < warmup; ++i) {
    spmm_rowsplit(ctx, n, d_ptr, d_ind, a_val, cols, b, c);
  }
  ctx.sync();
  EventSpan t;
  t.create(true);
  t.begin(ctx.stream);
  for (int32_t i = 0; i < repeat; ++i) {
    spmm_rowsplit(ctx, n, d_ptr, d_ind, a_val, cols, b, c);
  }
  t.end(ctx.stream);
  ctx.sync();
  *wall_ms = repeat > 0 ? t.ms() / repeat : 0.0f;
  t.destroy();
}

} // extern "C"
