#ifndef SPORDER_H
#define SPORDER_H

/*
 * sporder -- C ABI of the MI355X (gfx950) sparse-matrix reordering library
 * (libsporder_hip.so).
 *
 * Every entry point below keeps the name, argument list and struct layout of
 * the reference's C ABI (sporder/include/sporder.h of Siaaa-3/ChunkedGreedy;
 * each declaration cites the line it replaces), so an existing binding
 * (nanobind, ctypes, cgo, ...) links against this library unchanged.  Entry
 * points marked "(new)" have no counterpart there.
 *
 * Conventions shared by every entry point (reference sporder.h:13-41):
 *   - Synchronous: calls return only after device outputs and host
 *     out-parameters are ready.
 *   - d_-prefixed pointers are device memory on the context's device; all
 *     other pointers are host memory.
 *   - The library runs on a private HIP stream (created blocking, default
 *     priority), so inputs produced on another non-default stream must be
 *     synchronized by the caller first.
 *   - CSR patterns are square (n rows and columns), zero-based, with column
 *     indices sorted within each row.
 *   - Invalid arguments and HIP errors abort the process with a diagnostic on
 *     stderr (no return codes), as in the reference.
 *   - Permutations are in new2old form: d_new_order[p] = the original row
 *     that belongs in new position p.
 *   - Timing and stats pointers are optional (NULL to skip).
 *   - Scratch memory comes from a grow-only workspace owned by the context;
 *     steady-state calls of equal or smaller size allocate nothing.
 */

#include <stdbool.h>
#include <stdint.h>

#define SPORDER_API __attribute__((visibility("default")))

#ifdef __cplusplus
extern "C" {
#endif

typedef struct sporder_context_struct *sporder_context_t;

/* Context bound to the device current at creation; one thread at a time.
 * Reference: sporder.h:43-52. */
SPORDER_API sporder_context_t sporder_context_create(void);
SPORDER_API void sporder_context_destroy(sporder_context_t h);

/* Reference: sporder.h:54-58. */
typedef struct {
  int32_t k;
  float oversampling;
  int32_t max_rounds;
} sporder_options_t;

/* Reference: sporder.h:64-72. */
typedef struct {
  double wall_ms;
  float csr2csc_ms;
  float similarity_ms;
  float matching_ms;
  float advance_ms;
  float *matching_per_level_ms;
  float *advance_per_level_ms;
} sporder_hm_timing_t;

/* Reference: sporder.h:85-94. */
typedef struct {
  int32_t k_used;
  int32_t m_used;
  double avg_degree;
  double avg_edge_weight;
  int32_t zero_degree_rows;
  int32_t *level_size;
  int32_t *matched_pairs;
  int32_t *rounds;
} sporder_hm_stats_t;

/* Hierarchical matching.  Not built in this library (a different algorithm
 * from the Chunked Greedy path): the symbol exists for link compatibility and
 * aborts with a diagnostic.  Reference: sporder.h:119-123. */
SPORDER_API void sporder_hierarchical_matching(
    sporder_context_t ctx, int32_t n, int32_t nnz, const int32_t *d_ptr,
    const int32_t *d_ind, bool is_symmetric, int32_t num_levels,
    const sporder_options_t *opts, int32_t *d_new_order,
    sporder_hm_timing_t *timing, sporder_hm_stats_t *stats);

/* Reference: sporder.h:128-133. */
typedef struct {
  double wall_ms;
  float csr2csc_ms;
  float similarity_ms;
  float chunk_greedy_ms;
} sporder_cg_timing_t;

/* Reference: sporder.h:154-167. */
typedef struct {
  int32_t k_used;
  int32_t m_used;
  double avg_degree;
  double avg_edge_weight;
  int32_t zero_degree_rows;
  int32_t chunk_size_used;
  int32_t chain_restarts;
  double avg_followed_weight;
  double cut_weight_fraction;
} sporder_cg_stats_t;

/* Global-sketch chunk greedy (sporder-cg): the top-k table of the sketch over
 * all rows (one chunk of n rows), then the csg greedy chain per chunk of
 * chunk_size rows; cut_weight_fraction is the table weight leaving its chunk.
 * Defaults as csg.  Reference: sporder.h:176-182, sporder/src/cg/. */
SPORDER_API void sporder_chunk_greedy(sporder_context_t ctx, int32_t n,
                                      int32_t nnz, const int32_t *d_ptr,
                                      const int32_t *d_ind, bool is_symmetric,
                                      int32_t k, float oversampling,
                                      int32_t chunk_size, int32_t *d_new_order,
                                      sporder_cg_timing_t *timing,
                                      sporder_cg_stats_t *stats);

/* Reference: sporder.h:203-208. */
typedef struct {
  double wall_ms;
  float csr2csc_ms;
  float similarity_ms;
  float chunk_greedy_ms;
} sporder_csg_timing_t;

/* Reference: sporder.h:213-222. */
typedef struct {
  int32_t k_used;
  int32_t m_used;
  double avg_degree;
  double avg_edge_weight;
  int32_t zero_degree_rows;
  int32_t chunk_size_used;
  int32_t chain_restarts;
  double avg_followed_weight;
} sporder_csg_stats_t;

/*
 * Chunked Greedy reordering (sporder-csg).  Reference: sporder.h:224-228,
 * bridge sporder/src/sporder.cpp:140-166.
 *
 * Defaults: k <= 0 -> min(256, max(16, nnz / n)); oversampling <= 0 -> 4;
 * chunk_size <= 0 -> 1024.  Requires (int)(k * oversampling) <= 512.
 * Rows are cut into aligned chunks; each row's top-k Dice neighbours within
 * its chunk come from a 32-lane space-saving sketch of capacity
 * m = 32 * ceil((int)(k*oversampling) / 32); a greedy chain per chunk writes
 * d_new_order[start..end).  The output equals the reference's bit for bit.
 * is_symmetric says the pattern equals its transpose; the transpose is then
 * taken to be the CSR itself, as in the reference.
 */
SPORDER_API void sporder_chunk_similarity_greedy(
    sporder_context_t ctx, int32_t n, int32_t nnz, const int32_t *d_ptr,
    const int32_t *d_ind, bool is_symmetric, int32_t k, float oversampling,
    int32_t chunk_size, int32_t *d_new_order, sporder_csg_timing_t *timing,
    sporder_csg_stats_t *stats);

/* Reference: sporder.h:230-233. */
typedef enum {
  SPORDER_REORDER_ROWS = 0,
  SPORDER_REORDER_SYMMETRIC = 1,
} sporder_reorder_mode_t;

/*
 * Apply a new2old permutation: ROWS copies old row new_order[p] to row p;
 * SYMMETRIC also maps column c to old2new[c] and re-sorts each row (values
 * follow).  Reference: sporder.h:253-258, sporder/src/reorder.cu:72-149.
 */
SPORDER_API void
sporder_reorder(sporder_context_t ctx, int32_t n, int32_t nnz,
                const int32_t *d_ptr_old, const int32_t *d_ind_old,
                const float *d_val_old, const int32_t *d_new_order,
                sporder_reorder_mode_t mode, int32_t *d_ptr_new,
                int32_t *d_ind_new, float *d_val_new);

/* Pillar count: the number of distinct (window, column) pairs over windows of
 * `height` consecutive rows; height 1 gives nnz for a CSR without duplicates.
 * Reference: sporder.h:276-279, sporder/src/count_pillars.cu:11-85. */
SPORDER_API void sporder_count_pillars(sporder_context_t ctx, int32_t n,
                                       int32_t nnz, const int32_t *d_ptr,
                                       const int32_t *d_ind, int32_t height,
                                       int32_t *count);

/*
 * SpMM benchmark hook.  Same symbol and arguments as the reference
 * (sporder.h:295-299, sporder/src/bench_cusparse_spmm.cu:25-103); the kernel
 * timed is this library's CSR SpMM (row-split, fp32), not cuSPARSE.  A's
 * values and a row-major B are U(0,1] from Philox4x32-10 keyed by `seed`
 * (the reference used cuRAND XORWOW and a column-major B).  *wall_ms is the
 * mean time per repeat, measured with HIP events on the library stream.
 */
SPORDER_API void sporder_bench_cusparse_spmm(sporder_context_t ctx, int32_t n,
                                             int32_t nnz, const int32_t *d_ptr,
                                             const int32_t *d_ind, int32_t cols,
                                             int32_t warmup, int32_t repeat,
                                             uint64_t seed, float *wall_ms);

/* Reference: sporder.h:312-317. */
typedef struct {
  double wall_ms;
  float csr2csc_ms;
  float similarity_ms;
  float unpack_ms;
} sporder_sim_timing_t;

/* Reference: sporder.h:322-328. */
typedef struct {
  int32_t k_used;
  int32_t m_used;
  double avg_degree;
  double avg_edge_weight;
  int32_t zero_degree_rows;
} sporder_sim_stats_t;

/*
 * Global top-k Dice similarity graph from the space-saving sketch.
 * Defaults: k <= 0 -> min(32, max(16, 2 * (nnz / n))); oversampling <= 0 -> 2.
 * Computed by the same sketch kernel as the csg path with one chunk spanning
 * all rows.  Reference: sporder.h:330-335, sporder/src/similarity_graph.cu.
 */
SPORDER_API void sporder_similarity_graph(
    sporder_context_t ctx, int32_t n, int32_t nnz, const int32_t *d_ptr,
    const int32_t *d_ind, bool is_symmetric, int32_t k, float oversampling,
    int32_t *d_indices, float *d_weights, sporder_sim_timing_t *timing,
    sporder_sim_stats_t *stats);

/* Reference: sporder.h:353-360. */
typedef struct {
  double wall_ms;
  float csr2csc_ms;
  float spgemm_ms;
  float dice_ms;
  float sort_ms;
  float select_ms;
} sporder_sim_exact_timing_t;

/* Reference: sporder.h:365-371. */
typedef struct {
  int32_t k_used;
  int64_t c_nnz;
  double avg_degree;
  double avg_edge_weight;
  int32_t zero_degree_rows;
} sporder_sim_exact_stats_t;

/* Exact similarity via SpGEMM.  Not built (a validation tool resting on a
 * closed library in the reference): aborts with a diagnostic.
 * Reference: sporder.h:373-377. */
SPORDER_API void sporder_similarity_graph_exact(
    sporder_context_t ctx, int32_t n, int32_t nnz, const int32_t *d_ptr,
    const int32_t *d_ind, bool is_symmetric, int32_t k, int32_t *d_indices,
    float *d_weights, sporder_sim_exact_timing_t *timing,
    sporder_sim_exact_stats_t *stats);

/*
 * (new) The csg sketch table on its own: for each row, its top-k in-chunk
 * neighbours, d_indices/d_weights n*k, unused entries (-1, 0.0f).  k,
 * oversampling and chunk_size must be resolved (> 0).  This is the
 * reference's internal stage multi_chunk_similarity_top_k
 * (sporder/src/common/chunk_similarity_top_k.h:23-28), exported so the sketch
 * can be checked bit for bit.
 */
SPORDER_API void sporder_chunk_similarity_top_k(
    sporder_context_t ctx, int32_t n, int32_t nnz, const int32_t *d_ptr,
    const int32_t *d_ind, bool is_symmetric, int32_t k, float oversampling,
    int32_t chunk_size, int32_t *d_indices, float *d_weights);

/* (new) SpMM kernel variants. */
typedef enum {
  SPORDER_SPMM_AUTO = 0,     /* row-split with long rows in segments */
  SPORDER_SPMM_ROW_SPLIT = 1,
  SPORDER_SPMM_MERGE_PATH = 2,
} sporder_spmm_algo_t;

/*
 * (new) C = A * B for a CSR A (n x n, values d_val) and row-major dense
 * B (n x cols) and C (n x cols), fp32.  ROW_SPLIT (and AUTO) compute each
 * C element in a stated order, bit-exact with a CPU loop in that order:
 *   - a row with at most SPORDER_SPMM_LONG_ROW nonzeros:
 *     acc = fmaf(a_p, B[col_p][j], acc) over p in CSR order from 0.0f;
 *   - a longer row: segments of SPORDER_SPMM_SEGMENT nonzeros from the row's
 *     start, each such a chain from 0.0f, added left to right
 *     (((P0 + P1) + P2) + ...).
 * Long rows are spread over many waves, so one hub row does not serialise the
 * product.  MERGE_PATH splits rows at equal nonzero spans and adds the partial
 * sums with atomics, so it matches within rounding.  *kernel_ms (optional)
 * gets the time from HIP events on the library stream.  The reference
 * harness contract this serves is SpMMMethod.run
 * (bench/spmm/spmm_bench/base.py:48-59).
 */
#define SPORDER_SPMM_LONG_ROW 512
#define SPORDER_SPMM_SEGMENT 512
SPORDER_API void sporder_spmm_csr(sporder_context_t ctx, int32_t n,
                                  int32_t nnz, const int32_t *d_ptr,
                                  const int32_t *d_ind, const float *d_val,
                                  int32_t cols, const float *d_b, float *d_c,
                                  sporder_spmm_algo_t algo, float *kernel_ms);

/*
 * (new) C = diag(row_scale) A diag(col_scale) B with the row-split kernels.
 * It has no counterpart in the reference: it is for callers that scale the
 * product on both sides, such as a GCN's symmetric normalisation
 * D^-1/2 A D^-1/2, which the reference driver applies as two elementwise
 * products around the SpMM (experiments/e2e_gcn.py:117-123).  The column
 * scales come per nonzero, d_nz_col_scale[p] = col_scale[d_ind[p]] (nnz
 * floats, streamed beside d_val; a caller whose pattern does not change
 * computes it once), and d_row_scale holds n floats.  The B row gathered for
 * nonzero p is multiplied by d_nz_col_scale[p] (one fp32 multiply per
 * element) before its fmaf, and each finished row by its row scale, so the
 * result equals, bit for bit, B' = col_scale (.) B, C' = sporder_spmm_csr
 * ROW_SPLIT (A, B'), C = row_scale (.) C', without writing B' or C'.  Either
 * scale may be NULL (no scaling on that side).  Synchronous; *kernel_ms
 * (optional) as for sporder_spmm_csr.
 */
SPORDER_API void sporder_spmm_csr_scaled(sporder_context_t ctx, int32_t n,
                                         int32_t nnz, const int32_t *d_ptr,
                                         const int32_t *d_ind, const float *d_val,
                                         int32_t cols, const float *d_b,
                                         const float *d_row_scale,
                                         const float *d_nz_col_scale, float *d_c,
                                         float *kernel_ms);

/*
 * (new) SpMM plans.  The reference's SpMM harness converts each matrix once,
 * untimed, in SpMMMethod.prepare (bench/spmm/spmm_bench/base.py:41-46) and
 * times SpMMMethod.run; a plan is that conversion for this library's CSR
 * SpMM.  sporder_spmm_plan_create analyses a CSR pattern on the device in
 * blocks of 8 consecutive rows: a block's entries are the distinct columns of
 * its rows, each with the mask of rows holding it.  A tile of 64 rows whose
 * entries number at most half its nonzeros (rows that share columns:
 * bands, meshes in natural order, rows grouped by a reordering) is
 * "blocked": sporder_spmm_csr_plan computes each of its blocks with one load
 * of each entry's B row, applied to every row of the block that holds the
 * column.  Other tiles, tiles with a row past SPORDER_SPMM_LONG_ROW
 * nonzeros and tiles in which a row repeats a column (a CSR with duplicate
 * entries) run the row-split.  Entries are visited in ascending column
 * order, so the result is bit-identical to sporder_spmm_csr ROW_SPLIT (each C
 * element is the same fmaf chain in CSR order).  Blocks apply when cols is a
 * multiple of 64 and B and C are 16-byte aligned; otherwise the call is the
 * row-split.  The plan owns device memory on the context's device (8 bytes
 * per entry and 4 per block) until sporder_spmm_plan_destroy; it records n
 * and nnz, and the d_ptr/d_ind passed to a run must be the pattern it was
 * made from.
 */
typedef struct sporder_spmm_plan_struct *sporder_spmm_plan_t;
typedef struct {
  int32_t tiles;         /* tiles of 64 rows */
  int32_t blocked_tiles; /* tiles computed in blocks of 8 rows */
  int64_t blocked_rows;
  int64_t blocked_nnz;
  int64_t entries;       /* (column, row mask) entries of the blocked tiles */
} sporder_spmm_plan_info_t;

SPORDER_API sporder_spmm_plan_t sporder_spmm_plan_create(sporder_context_t ctx, int32_t n,
                                                         int32_t nnz, const int32_t *d_ptr,
                                                         const int32_t *d_ind,
                                                         sporder_spmm_plan_info_t *info);
SPORDER_API void sporder_spmm_plan_destroy(sporder_spmm_plan_t plan);
SPORDER_API void sporder_spmm_csr_plan(sporder_context_t ctx, sporder_spmm_plan_t plan,
                                       int32_t n, int32_t nnz, const int32_t *d_ptr,
                                       const int32_t *d_ind, const float *d_val,
                                       int32_t cols, const float *d_b, float *d_c,
                                       float *kernel_ms);

/*
 * (new) HBM ceiling.  No counterpart in the reference, whose SpMM hook times
 * its kernel with events on the library stream
 * (sporder/src/bench_cusparse_spmm.cu:51-100); this times a pure read, a pure
 * write or a copy of `bytes` (a multiple of 16) with this library's own
 * streaming kernels (16 bytes per lane per access, each workgroup a contiguous
 * 16 KiB span, spans in contiguous runs per XCD), with ordinary or
 * non-temporal accesses, so that the HBM-bound kernels' roofline fractions
 * can be read against the rate streaming code reaches on the device.  One
 * untimed launch, then `iters` timed ones; *ms_per_launch (optional) gets
 * their mean.  READ leaves d_dst (16-byte aligned, at least 16 bytes) as it
 * was; WRITE fills d_dst with the float 1.0f; COPY copies d_src to d_dst
 * (non-overlapping).  Synchronous.
 */
typedef enum {
  SPORDER_STREAM_READ = 0,
  SPORDER_STREAM_WRITE = 1,
  SPORDER_STREAM_COPY = 2
} sporder_stream_op_t;
SPORDER_API void sporder_hbm_stream(sporder_context_t ctx, int32_t op, int32_t nontemporal,
                                    void *d_dst, const void *d_src, int64_t bytes,
                                    int32_t iters, float *ms_per_launch);

/*
 * (new) sporder_spmm_csr (ROW_SPLIT) that allocates nothing.  It has no
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory (tight serving loops, harnesses that forbid hipMalloc).  It runs
 * eagerly on the library's private stream, reads a count back to the host
 * partway and ends with a synchronize, so it cannot be recorded into a HIP
 * graph.  The result equals sporder_spmm_csr's bit for bit (same
 * kernels, same stated order).  The caller passes every input and output; the
 * scratch the row-split needs for rows past SPORDER_SPMM_LONG_ROW nonzeros
 * (a 16-byte descriptor per such row, 4 bytes per segment and a partial row of
 * `cols` floats per segment, each part rounded up to 256 bytes) comes from a
 * static device array of SPORDER_SPMM_NOALLOC_SCRATCH_BYTES that each GPU
 * holds from the first context created on it until the process ends.  Every
 * call on one GPU shares that array: calls from one process on one GPU are
 * serialised by a lock held for the whole call; calls that overlap from two
 * processes on one GPU each use their own process's array.
 * Returns 0 when C is written, or SPORDER_SPMM_NOALLOC_TOO_LARGE (nothing
 * computed) when the input's long rows need more scratch than the array
 * holds.  Invalid arguments abort, as elsewhere.  Synchronous.
 */
#define SPORDER_SPMM_NOALLOC_SCRATCH_BYTES (64u << 20)
#define SPORDER_SPMM_NOALLOC_TOO_LARGE 1
SPORDER_API int32_t sporder_spmm_csr_noalloc(sporder_context_t ctx, int32_t n,
                                             int32_t nnz, const int32_t *d_ptr,
                                             const int32_t *d_ind, const float *d_val,
                                             int32_t cols, const float *d_b, float *d_c);

#ifdef __cplusplus
}
#endif

#endif /* SPORDER_H */
