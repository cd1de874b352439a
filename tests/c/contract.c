/*
 * contract.c -- C99 contract check of libsporder_hip.so.
 *
 * The reference guards its C ABI with a C program linked against the library
 * and run as a CTest (sporder/tests/smoke.c:55-130, sporder/CMakeLists.txt:
 * 69-82): the header must compile as plain C and the library must link into
 * and run from a C program.  This program does the same for this library and
 * checks each result: every exported entry point that is built is called at
 * least once (the two that abort by design, hierarchical matching and exact
 * SpGEMM similarity, are not), on a band matrix |i - j| <= 2 of n = 1000 rows.
 *
 * Checks: permutations are permutations of 0..n-1 and agree between calls
 * with and without timing/statistics; the csg statistics carry the resolved
 * defaults; the pillar count at height 1 equals nnz after a row permutation;
 * the symmetric permutation apply equals P A P^T computed here; row 0 of the
 * similarity graph is the known answer 1, 2, 3, 4 (first weight three
 * sequential fp32 adds of 2/7: bits 0x3f5b6db8); the csg sketch table with
 * one chunk equals the similarity graph; the row-split SpMM equals a C loop
 * in the stated fmaf order bit for bit; merge-path is within 1e-5 of it.
 *
 * Exit status 0 and "contract: OK" on success; otherwise the first failed
 * check is printed and the status is 1.
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <sporder.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define HIPCHK(call)                                                           \
  do {                                                                         \
    hipError_t e_ = (call);                                                    \
    if (e_ != hipSuccess) {                                                    \
      fprintf(stderr, "%s:%d: HIP error %s\n", __FILE__, __LINE__,            \
              hipGetErrorString(e_));                                          \
      return 1;                                                                \
    }                                                                          \
  } while (0)

#define CHECK(cond, what)                                                      \
  do {                                                                         \
    if (!(cond)) {                                                             \
      fprintf(stderr, "contract: FAILED: %s\n", what);                         \
      return 1;                                                                \
    }                                                                          \
    printf("contract: ok: %s\n", what);                                        \
  } while (0)

static int is_permutation(const int32_t *p, int32_t n) {
  char *seen = calloc((size_t)n, 1);
  int ok = seen != NULL;
  for (int32_t i = 0; ok && i < n; ++i) {
    ok = p[i] >= 0 && p[i] < n && !seen[p[i]];
    if (ok) seen[p[i]] = 1;
  }
  free(seen);
  return ok;
}

static uint32_t float_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, sizeof u);
  return u;
}

/* Host copy of a device int32 array. */
static int32_t *fetch_i32(const int32_t *d, size_t count) {
  int32_t *h = malloc(count * sizeof(int32_t) + 1);
  if (h != NULL && hipMemcpy(h, d, count * sizeof(int32_t), hipMemcpyDeviceToHost) != hipSuccess) {
    free(h);
    h = NULL;
  }
  return h;
}

int main(void) {
  const int32_t n = 1000, N = 32;
  int32_t *h_ptr = malloc((size_t)(n + 1) * sizeof(int32_t));
  int32_t *h_ind = malloc((size_t)n * 5 * sizeof(int32_t));
  float *h_val = malloc((size_t)n * 5 * sizeof(float));
  int32_t nnz = 0;
  h_ptr[0] = 0;
  for (int32_t i = 0; i < n; ++i) {
    for (int32_t j = i - 2; j <= i + 2; ++j) {
      if (j < 0 || j >= n) continue;
      h_ind[nnz] = j;
      h_val[nnz] = 0.25f + (float)((i * 7 + j * 3) % 11) * 0.125f;
      ++nnz;
    }
    h_ptr[i + 1] = nnz;
  }
  float *h_b = malloc((size_t)n * N * sizeof(float));
  for (int32_t i = 0; i < n * N; ++i) h_b[i] = (float)((i * 37) % 101 - 50) / 64.0f;

  int32_t *d_ptr, *d_ind, *d_order, *d_order2, *d_ptr2, *d_ind2, *d_idx, *d_idx2;
  float *d_val, *d_val2, *d_w, *d_w2, *d_b, *d_c;
  const int32_t k = 8;
  HIPCHK(hipMalloc((void **)&d_ptr, (size_t)(n + 1) * sizeof(int32_t)));
  HIPCHK(hipMalloc((void **)&d_ind, (size_t)nnz * sizeof(int32_t)));
  HIPCHK(hipMalloc((void **)&d_val, (size_t)nnz * sizeof(float)));
  HIPCHK(hipMalloc((void **)&d_order, (size_t)n * sizeof(int32_t)));
  HIPCHK(hipMalloc((void **)&d_order2, (size_t)n * sizeof(int32_t)));
  HIPCHK(hipMalloc((void **)&d_ptr2, (size_t)(n + 1) * sizeof(int32_t)));
  HIPCHK(hipMalloc((void **)&d_ind2, (size_t)nnz * sizeof(int32_t)));
  HIPCHK(hipMalloc((void **)&d_val2, (size_t)nnz * sizeof(float)));
  HIPCHK(hipMalloc((void **)&d_idx, (size_t)n * k * sizeof(int32_t)));
  HIPCHK(hipMalloc((void **)&d_idx2, (size_t)n * k * sizeof(int32_t)));
  HIPCHK(hipMalloc((void **)&d_w, (size_t)n * k * sizeof(float)));
  HIPCHK(hipMalloc((void **)&d_w2, (size_t)n * k * sizeof(float)));
  HIPCHK(hipMalloc((void **)&d_b, (size_t)n * N * sizeof(float)));
  HIPCHK(hipMalloc((void **)&d_c, (size_t)n * N * sizeof(float)));
  HIPCHK(hipMemcpy(d_ptr, h_ptr, (size_t)(n + 1) * sizeof(int32_t), hipMemcpyHostToDevice));
  HIPCHK(hipMemcpy(d_ind, h_ind, (size_t)nnz * sizeof(int32_t), hipMemcpyHostToDevice));
  HIPCHK(hipMemcpy(d_val, h_val, (size_t)nnz * sizeof(float), hipMemcpyHostToDevice));
  HIPCHK(hipMemcpy(d_b, h_b, (size_t)n * N * sizeof(float), hipMemcpyHostToDevice));

  sporder_context_t ctx = sporder_context_create();
  CHECK(ctx != NULL, "sporder_context_create returns a context");

  /* csg with every diagnostic, then with none: same permutation. */
  sporder_csg_timing_t ct;
  sporder_csg_stats_t cs;
  memset(&ct, 0, sizeof ct);
  memset(&cs, 0, sizeof cs);
  sporder_chunk_similarity_greedy(ctx, n, nnz, d_ptr, d_ind, true, 0, 0.0f, 0, d_order, &ct,
                                  &cs);
  int32_t *order = fetch_i32(d_order, (size_t)n);
  CHECK(order != NULL && is_permutation(order, n), "csg new_order is a permutation");
  CHECK(cs.k_used == 16 && cs.m_used == 64 && cs.chunk_size_used == 1024,
        "csg stats carry the resolved defaults (k 16, m 64, chunk 1024)");
  CHECK(ct.wall_ms >= (double)ct.chunk_greedy_ms && ct.chunk_greedy_ms >= 0.0f,
        "csg timing: wall covers the chain span");
  CHECK(cs.zero_degree_rows == 0 && cs.avg_degree > 0.0, "csg stats: every band row has neighbours");
  sporder_chunk_similarity_greedy(ctx, n, nnz, d_ptr, d_ind, true, 0, 0.0f, 0, d_order2, NULL,
                                  NULL);
  int32_t *order2 = fetch_i32(d_order2, (size_t)n);
  CHECK(order2 != NULL && memcmp(order, order2, (size_t)n * sizeof(int32_t)) == 0,
        "csg without diagnostics gives the same permutation");
  free(order2);

  /* cg */
  sporder_cg_stats_t gs;
  memset(&gs, 0, sizeof gs);
  sporder_chunk_greedy(ctx, n, nnz, d_ptr, d_ind, true, 0, 0.0f, 250, d_order2, NULL, &gs);
  order2 = fetch_i32(d_order2, (size_t)n);
  CHECK(order2 != NULL && is_permutation(order2, n), "cg new_order is a permutation");
  CHECK(gs.cut_weight_fraction >= 0.0 && gs.cut_weight_fraction <= 1.0,
        "cg cut_weight_fraction in [0, 1]");
  free(order2);

  /* ROWS apply, then the pillar count at height 1 is nnz. */
  sporder_reorder(ctx, n, nnz, d_ptr, d_ind, NULL, d_order, SPORDER_REORDER_ROWS, d_ptr2, d_ind2,
                  NULL);
  int32_t pillars = -1;
  sporder_count_pillars(ctx, n, nnz, d_ptr2, d_ind2, 1, &pillars);
  CHECK(pillars == nnz, "count_pillars(height 1) == nnz after a row permutation");
  sporder_count_pillars(ctx, n, nnz, d_ptr, d_ind, 1000, &pillars);
  CHECK(pillars == n, "count_pillars(height n) == n (every column once)");

  /* SYMMETRIC apply with values against P A P^T computed here. */
  sporder_reorder(ctx, n, nnz, d_ptr, d_ind, d_val, d_order, SPORDER_REORDER_SYMMETRIC, d_ptr2,
                  d_ind2, d_val2);
  {
    int32_t *p2 = fetch_i32(d_ptr2, (size_t)n + 1), *i2 = fetch_i32(d_ind2, (size_t)nnz);
    float *v2 = malloc((size_t)nnz * sizeof(float));
    int32_t *old2new = malloc((size_t)n * sizeof(int32_t));
    int ok = p2 != NULL && i2 != NULL && v2 != NULL && old2new != NULL &&
             hipMemcpy(v2, d_val2, (size_t)nnz * sizeof(float), hipMemcpyDeviceToHost) == hipSuccess;
    for (int32_t p = 0; ok && p < n; ++p) old2new[order[p]] = p;
    for (int32_t p = 0; ok && p < n; ++p) {
      const int32_t r = order[p], len = h_ptr[r + 1] - h_ptr[r];
      ok = p2[p + 1] - p2[p] == len;
      for (int32_t q = p2[p]; ok && q < p2[p + 1]; ++q) {
        ok = q == p2[p] || i2[q - 1] < i2[q]; /* sorted */
        int found = 0;
        for (int32_t e = h_ptr[r]; ok && e < h_ptr[r + 1]; ++e) {
          if (old2new[h_ind[e]] == i2[q]) {
            found = float_bits(h_val[e]) == float_bits(v2[q]);
          }
        }
        ok = ok && found;
      }
    }
    CHECK(ok, "reorder SYMMETRIC with values equals P A P^T");
    free(p2);
    free(i2);
    free(v2);
    free(old2new);
  }

  /* Similarity graph known answer, and the csg table with one chunk. */
  sporder_sim_stats_t ss;
  sporder_similarity_graph(ctx, n, nnz, d_ptr, d_ind, true, k, 4.0f, d_idx, d_w, NULL, &ss);
  {
    int32_t row0[8];
    float w0[8];
    HIPCHK(hipMemcpy(row0, d_idx, sizeof row0, hipMemcpyDeviceToHost));
    HIPCHK(hipMemcpy(w0, d_w, sizeof w0, hipMemcpyDeviceToHost));
    CHECK(row0[0] > 0 && row0[0] < n, "similarity_graph: row 0 has a valid best neighbour");
    CHECK(row0[0] == 1 && row0[1] == 2 && row0[2] == 3 && row0[3] == 4 && row0[4] == -1,
          "similarity_graph: row 0 neighbours are 1, 2, 3, 4");
    CHECK(float_bits(w0[0]) == 0x3f5b6db8u && w0[1] == 0.75f && w0[2] == 0.5f && w0[3] == 0.25f,
          "similarity_graph: row 0 weights are the sequential fp32 sums");
  }
  sporder_chunk_similarity_top_k(ctx, n, nnz, d_ptr, d_ind, true, k, 4.0f, n, d_idx2, d_w2);
  {
    int32_t *a = fetch_i32(d_idx, (size_t)n * k), *b = fetch_i32(d_idx2, (size_t)n * k);
    int32_t *wa = fetch_i32((const int32_t *)d_w, (size_t)n * k);
    int32_t *wb = fetch_i32((const int32_t *)d_w2, (size_t)n * k);
    CHECK(a && b && wa && wb && memcmp(a, b, (size_t)n * k * 4) == 0 &&
              memcmp(wa, wb, (size_t)n * k * 4) == 0,
          "chunk_similarity_top_k with one chunk equals similarity_graph");
    free(a);
    free(b);
    free(wa);
    free(wb);
  }

  /* SpMM: row-split against the stated fmaf order, AUTO equal, merge-path close. */
  {
    float *ref = malloc((size_t)n * N * sizeof(float)), *c = malloc((size_t)n * N * sizeof(float));
    for (int32_t i = 0; i < n; ++i) {
      for (int32_t j = 0; j < N; ++j) {
        float acc = 0.0f;
        for (int32_t p = h_ptr[i]; p < h_ptr[i + 1]; ++p) {
          acc = fmaf(h_val[p], h_b[(size_t)h_ind[p] * N + j], acc);
        }
        ref[(size_t)i * N + j] = acc;
      }
    }
    float ms = -1.0f;
    sporder_spmm_csr(ctx, n, nnz, d_ptr, d_ind, d_val, N, d_b, d_c, SPORDER_SPMM_ROW_SPLIT, &ms);
    HIPCHK(hipMemcpy(c, d_c, (size_t)n * N * sizeof(float), hipMemcpyDeviceToHost));
    CHECK(ms >= 0.0f && memcmp(c, ref, (size_t)n * N * sizeof(float)) == 0,
          "spmm_csr ROW_SPLIT equals the stated fmaf order bit for bit");
    sporder_spmm_csr(ctx, n, nnz, d_ptr, d_ind, d_val, N, d_b, d_c, SPORDER_SPMM_AUTO, NULL);
    HIPCHK(hipMemcpy(c, d_c, (size_t)n * N * sizeof(float), hipMemcpyDeviceToHost));
    CHECK(memcmp(c, ref, (size_t)n * N * sizeof(float)) == 0, "spmm_csr AUTO equals ROW_SPLIT");
    sporder_spmm_csr(ctx, n, nnz, d_ptr, d_ind, d_val, N, d_b, d_c, SPORDER_SPMM_MERGE_PATH, NULL);
    HIPCHK(hipMemcpy(c, d_c, (size_t)n * N * sizeof(float), hipMemcpyDeviceToHost));
    int close = 1;
    for (int32_t i = 0; i < n * N; ++i) {
      close = close && fabsf(c[i] - ref[i]) <= 1e-5f * (fabsf(ref[i]) + 1.0f);
    }
    CHECK(close, "spmm_csr MERGE_PATH within 1e-5 of the stated order");
    free(ref);
    free(c);
  }
  float bench_ms = -1.0f;
  sporder_bench_cusparse_spmm(ctx, n, nnz, d_ptr, d_ind, N, 1, 3, 7u, &bench_ms);
  CHECK(bench_ms > 0.0f, "bench_cusparse_spmm reports a positive mean time");

  sporder_context_destroy(ctx);
  free(order);
  hipFree(d_ptr);
  hipFree(d_ind);
  hipFree(d_val);
  hipFree(d_order);
  hipFree(d_order2);
  hipFree(d_ptr2);
  hipFree(d_ind2);
  hipFree(d_val2);
  hipFree(d_idx);
  hipFree(d_idx2);
  hipFree(d_w);
  hipFree(d_w2);
  hipFree(d_b);
  hipFree(d_c);
  free(h_ptr);
  free(h_ind);
  free(h_val);
  free(h_b);
  printf("contract: OK\n");
  return 0;
}
