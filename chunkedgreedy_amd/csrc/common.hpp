// common.hpp -- runtime pieces shared by every kernel file of
// libsporder_hip.so: error handling (abort with a diagnostic, as the
// reference's ensure/expect do, sporder/src/common/error_checking.h:12-61),
// the context (private stream + device facts + grow-only workspace; the
// reference's counterpart is sporder/src/common/context.h:67-197), event
// timers (sporder/src/common/timer.h:12-51) and wave64 helpers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstdlib>

#include "sporder.h"

namespace sporder_hip {

[[noreturn]] void fail_hip(hipError_t err, const char *expr, const char *file,
                           int line);
[[noreturn]] void fail_expect(const char *msg, const char *file, int line);

#define SP_HIP(expr)                                                           \
  do {                                                                         \
    hipError_t sp_err_ = (expr);                                               \
    if (sp_err_ != hipSuccess) {                                               \
      ::sporder_hip::fail_hip(sp_err_, #expr, __FILE__, __LINE__);             \
    }                                                                          \
  } while (0)

#define SP_EXPECT(cond, msg)                                                   \
  do {                                                                         \
    if (!(cond)) {                                                             \
      ::sporder_hip::fail_expect(msg, __FILE__, __LINE__);                     \
    }                                                                          \
  } while (0)

#define SP_LAUNCH_CHECK() SP_HIP(hipGetLastError())

constexpr int kWave = 64;

__host__ __device__ inline int64_t ceil_div64(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Bump allocator over a grow-only device buffer owned by the context.
// reserve() must be called with the call's total before any take().
struct Workspace {
  void *base = nullptr;
  size_t capacity = 0;
  size_t offset = 0;

  static size_t align(size_t bytes) { return (bytes + 255u) & ~size_t(255u); }
};

struct Context {
  int device = 0;
  hipStream_t stream = nullptr;
  int num_cus = 0;
  int max_threads_per_cu = 0;
  size_t lds_per_block = 0;
  Workspace ws;
  Workspace aux; // second grow-only buffer, for temporaries sized mid-call
  // Three more streams (default priority) for independent kernels of one
  // call, forked from and joined back into `stream` with the events below, so
  // a synchronize of `stream` also waits for their work.  The four are the
  // last of kMadeStreams streams made at init (make_streams: the earlier ones
  // ran the side streams' kernels one after another in some processes).
  hipStream_t side[3] = {};
  static constexpr int kMadeStreams = 8;
  hipStream_t unused_streams[kMadeStreams - 4] = {};
  hipEvent_t fork_ev = nullptr;
  hipEvent_t join_ev[3] = {};
  hipEvent_t prep_ev = nullptr; // a stage's preparation done (csg's global path)
  // Pinned host words for small device-to-host readbacks.
  int32_t *host_words = nullptr;
  static constexpr int kHostWords = 16;

  void init();
  void destroy();
  void make_streams();
  void sync() { SP_HIP(hipStreamSynchronize(stream)); }

  // Grow the workspace to hold `bytes` (rounded), then reset the cursor.
  void reserve(size_t bytes);
  // Base of the auxiliary buffer grown to at least `bytes`, for temporaries
  // whose size is only known after part of a call has run (the main
  // workspace's earlier takes stay valid).
  void *aux_reserve(size_t bytes);
  template <typename T> T *take(size_t count) {
    size_t bytes = Workspace::align(count * sizeof(T) + (count == 0 ? 1 : 0));
    SP_EXPECT(ws.offset + bytes <= ws.capacity,
              "workspace overflow (internal sizing error)");
    T *p = reinterpret_cast<T *>(static_cast<char *>(ws.base) + ws.offset);
    ws.offset += bytes;
    return p;
  }
  // Blocks for a grid-stride kernel: at least `min_blocks`, at most what
  // `waves` full passes of the device at `block` threads per block holds.
  int grid_for(int64_t work_blocks, int block, int waves = 4) const {
    int64_t cap = static_cast<int64_t>(num_cus) * max_threads_per_cu * waves /
                  block;
    if (cap < 1) cap = 1;
    int64_t g = work_blocks < cap ? work_blocks : cap;
    return static_cast<int>(g < 1 ? 1 : g);
  }
};

// Makes the work already queued on ctx.stream a prerequisite of side[i]
// (fork) and the work queued on side[i] a prerequisite of ctx.stream (join).
void fork_side(Context &ctx, int i);
void join_side(Context &ctx, int i);

// Routes the context's launches (which use ctx.stream) to `s` for the guard's
// lifetime.  Code run under it must not synchronize or grow the workspace.
struct OnStream {
  Context &ctx;
  hipStream_t saved;
  OnStream(Context &c, hipStream_t s) : ctx(c), saved(c.stream) { c.stream = s; }
  ~OnStream() { ctx.stream = saved; }
  OnStream(const OnStream &) = delete;
  OnStream &operator=(const OnStream &) = delete;
};

// Bytes a workspace request of `count` T's occupies (for reserve sums).
template <typename T> inline size_t ws_bytes(size_t count) {
  return Workspace::align(count * sizeof(T) + (count == 0 ? 1 : 0));
}

// One timed span on the library stream (begin/end are stream-ordered).
struct EventSpan {
  hipEvent_t a = nullptr, b = nullptr;
  bool on = false;
  void create(bool enable) {
    on = enable;
    if (on) {
      SP_HIP(hipEventCreate(&a));
      SP_HIP(hipEventCreate(&b));
    }
  }
  void begin(hipStream_t s) {
    if (on) SP_HIP(hipEventRecord(a, s));
  }
  void end(hipStream_t s) {
    if (on) SP_HIP(hipEventRecord(b, s));
  }
  float ms() const {
    float t = 0.0f;
    if (on) SP_HIP(hipEventElapsedTime(&t, a, b));
    return t;
  }
  void destroy() {
    if (on) {
      SP_HIP(hipEventDestroy(a));
      SP_HIP(hipEventDestroy(b));
      on = false;
    }
  }
};

// ---- host-side stages shared between files -------------------------------

// Takes, with `device` current, that device's address of the no-allocation
// SpMM scratch (spmm.hip); called once per context creation.
void spmm_noalloc_setup(int device);

// Rows of a tile of an SpMM plan (spmm_plan.hip); row-split tile lists count
// in these units.
constexpr int kSpmmTileRows = 64;

// Row-split SpMM in the stated order over the listed tiles (every row when
// `tiles` is null), long rows in segments; reserves the context workspace.
// long_rows false: the caller knows that no row passes SPORDER_SPMM_LONG_ROW
// nonzeros, and the long-row workspace and launches are left out.
void spmm_rowsplit_tiles(Context &ctx, int32_t n, int32_t nnz, const int32_t *ptr,
                         const int32_t *ind, const float *val, int32_t N, const float *B,
                         float *C, const int32_t *tiles, int64_t ntiles, bool long_rows = true);

// In-place exclusive (inclusive=false) or inclusive scan of `count` int32
// values; `tmp` must hold scan_tmp_elems(count) int32.
size_t scan_tmp_elems(int64_t count);
void scan_i32(Context &ctx, const int32_t *in, int32_t *out, int64_t count,
              bool inclusive, int32_t *tmp);
// The same scan when totals[t] already holds the sum of elements
// [t * kScanTileElems, (t + 1) * kScanTileElems) (totals sized as `tmp`
// above; overwritten).
constexpr int kScanTileElems = 4096;
void scan_i32_from_totals(Context &ctx, const int32_t *in, int32_t *out, int64_t count,
                          bool inclusive, int32_t *totals);

// Stable LSD radix sort of (key, value) pairs on the low `key_bits` bits.
// Input in keys_in/vals_in (preserved), result in keys_out/vals_out; the
// alt buffers are ping-pong space of `count` elements each; `tmp` must hold
// radix_tmp_elems(count) int32.
size_t radix_tmp_elems(int64_t count);
void radix_sort_pairs(Context &ctx, const uint32_t *keys_in,
                      const uint32_t *vals_in, uint32_t *keys_out,
                      uint32_t *vals_out, uint32_t *keys_alt,
                      uint32_t *vals_alt, int64_t count, int key_bits,
                      int32_t *tmp);

// Stable CSR -> CSC transpose (rows ascending within each column).
// Workspace needed: csr2csc_ws_bytes(n, nnz).
size_t csr2csc_ws_bytes(int32_t n, int32_t nnz);
void csr2csc(Context &ctx, int32_t n, int32_t nnz, const int32_t *d_ptr,
             const int32_t *d_ind, int32_t *d_col_ptr, int32_t *d_row_ind);

// Chunk-restricted sketch + top-k table (u64 weighted_index, n*k) from the
// global CSC.  With d_chunks non-null only the rows of the chunks listed in
// d_chunks[0 .. *d_chunk_count) are computed.  `prepared`, when given, is
// recorded once the run search is done and before the sketch launch.
// d_row_valid, when given, receives each computed row's number of valid table
// entries (the non-empty prefix of its table row, written with the row); rows
// not computed are left as they are.  `host_list_len`, when known
// (>= 2) and d_chunks is given, lets the first listed chunk (the largest
// size class) have its run search and sketch first while the other chunks'
// run search runs beside it on side stream 2 (joined back before return).
// Must be called with ctx.stream = side[0] or the library stream, not side[2].
size_t chunk_sketch_ws_bytes(int32_t n, int32_t nnz, int32_t chunk_size);
void chunk_sketch_top_k(Context &ctx, int32_t n, int32_t nnz, int32_t k, int32_t chunk_size,
                        int32_t m_capacity, const int32_t *d_ptr,
                        const int32_t *d_ind, const int32_t *d_col_ptr,
                        const int32_t *d_row_ind, uint64_t *d_table,
                        const int32_t *d_chunks = nullptr,
                        const int32_t *d_chunk_count = nullptr,
                        hipEvent_t prepared = nullptr, int32_t *d_row_valid = nullptr,
                        int64_t host_list_len = -1);
// The is_symmetric mirror check of the rows chunk_sketch_top_k computes for
// the same list: mirror_term (below) of each of their nonzeros, added into
// *mirror.  Independent of the sketch; the caller runs it where it holds back
// nothing.
void chunk_mirror_check(Context &ctx, int32_t n, int32_t chunk_size, const int32_t *d_ptr,
                        const int32_t *d_ind, const int32_t *d_chunks,
                        const int32_t *d_chunk_count, int64_t host_list_len,
                        unsigned long long *mirror);

// Chunk-local variant: one workgroup per chunk with the chunk's transpose in
// LDS.  Applicable when chunk_local_supported(n, chunk_size).
// chunk_local_classify fills d_lists (3*num_chunks int32) and d_counts (4
// int32): the chunks of LDS tier 2 in d_lists[0 .. d_counts[0]), the chunks
// too large for LDS in d_lists[num_chunks .. num_chunks + d_counts[1]) (for
// chunk_sketch_top_k over the global CSC; with is_symmetric, the largest
// chunks that tier 2 could hold go there as well, to run beside it), the
// tier-1 chunks in d_lists[2 num_chunks .. 2 num_chunks + d_counts[2]), and
// d_counts[3] = 0, the counter tier 2 claims its chunks from (so each tier-2
// launch needs a classification before it).  chunk_local_sketch_top_k then
// writes the rows of tier-1 chunks (tiers & 1; chunk_size <= 1024) and of the
// listed tier-2 chunks (tiers & 2); the two launches are independent and may
// run on different streams.  With t1_list_len >= 0 (d_counts[2], read back)
// tier 1 runs over its list with at most that many workgroups, else one per
// chunk.  d_row_valid as for chunk_sketch_top_k.
constexpr int kLocalRowCap = 4096;
bool chunk_local_supported(int32_t n, int32_t chunk_size);
void chunk_local_classify(Context &ctx, int32_t n, int32_t chunk_size, const int32_t *d_ptr,
                          int32_t *d_lists, int32_t *d_counts, bool is_symmetric);
void chunk_local_sketch_top_k(Context &ctx, int32_t n, int32_t k, int32_t chunk_size,
                              int32_t m_capacity, const int32_t *d_ptr, const int32_t *d_ind,
                              uint64_t *d_table, const int32_t *d_lists,
                              int32_t *d_counts, int tiers,
                              int32_t *d_row_valid = nullptr,
                              unsigned long long *mirror = nullptr,
                              int64_t t1_list_len = -1);

// Degree / weight totals of a top-k table (reference
// sporder/src/common/similarity_top_k.cu:120-172).
struct TopKTotals {
  unsigned long long total_degree;
  double total_weight;
  int32_t zero_degree_rows;
  int32_t pad;
};
void top_k_stats(Context &ctx, int32_t n, int32_t k, const uint64_t *d_table,
                 TopKTotals *d_totals);

int bits_for(int64_t max_value);

// Set `count` u32 words to `value` with a kernel on the library stream
// (a kernel rather than a memset node, so a captured call stays correct).
void fill_u32(Context &ctx, void *p, int64_t count, uint32_t value);

// ---- device helpers --------------------------------------------------------

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Workgroup index remapped so that each XCD takes a contiguous run of the
// grid: the dispatcher hands workgroups to the kXcds XCDs round-robin, so
// workgroup g runs on XCD g % kXcds; neighbouring work (rows that share B
// rows, say) then shares that XCD's L2.  A bijection of [0, gridDim.x).
constexpr int kXcds = 8;
__device__ __forceinline__ int64_t xcd_block() {
  const int64_t G = gridDim.x, q = G / kXcds, rem = G % kXcds, x = blockIdx.x % kXcds;
  return x * q + (x < rem ? x : rem) + blockIdx.x / kXcds;
}

// Workgroup index remapped so that each run of W consecutive logical
// workgroups (a tile of rows) stays on one XCD and the tiles are dealt to the
// XCDs in turn: XCD x takes tiles x, x + kXcds, x + 2 kXcds, ...  Rows of one
// tile share that XCD's L2, and work that grows or shrinks along the index
// (hubs first in a degree-sorted graph) is spread over every XCD.  The grid
// past the last whole round of kXcds tiles keeps its own index.  A bijection
// of [0, gridDim.x).
__device__ __forceinline__ int64_t xcd_tile_block(int64_t W) {
  const int64_t G = gridDim.x, g = blockIdx.x;
  const int64_t full = (G / (kXcds * W)) * (kXcds * W);
  if (g >= full) return g;
  const int64_t x = g % kXcds, i = g / kXcds;
  return ((i / W) * kXcds + x) * W + i % W;
}

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

// Orders a wave's LDS accesses: what one lane wrote before is visible to
// every lane of the wave after.
__device__ __forceinline__ void wave_lds_order() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// A wave-uniform mask with bit i (wave-uniform) cleared: one s_bitset0,
// where mask &= mask - 1 takes a 64-bit subtract and an and.  readfirstlane
// states the uniformity to the compiler, which drops it where it already
// holds both in scalar registers.
__device__ __forceinline__ uint64_t clear_bit(uint64_t mask, int i) {
  uint64_t m =
      static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int32_t>(mask))) |
      (static_cast<uint64_t>(static_cast<uint32_t>(
           __builtin_amdgcn_readfirstlane(static_cast<int32_t>(mask >> 32))))
       << 32);
  const int32_t b = __builtin_amdgcn_readfirstlane(i);
  asm("s_bitset0_b64 %0, %1" : "+s"(m) : "s"(b));
  return m;
}

__device__ __forceinline__ int32_t readlane(int32_t v, int lane) {
  return __builtin_amdgcn_readlane(v, lane);
}
__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// ---- wave64 reductions and scans on DPP --------------------------------------
//
// GFX9 data-parallel primitives move values between lanes inside the VALU
// (a few cycles), where __shfl* goes through ds_bpermute (LDS latency).
// Controls: quad_perm 0xB1 = [1,0,3,2], 0x4E = [2,3,0,1]; 0x141 row_half_mirror;
// 0x140 row_mirror; 0x111.. row_shr:n (0x110 + n); 0x142 row_bcast:15 (lane 15
// of each row to the next row, rows selected by row_mask 0xa); 0x143
// row_bcast:31 (lane 31 to rows 2 and 3, row_mask 0xc).  Lanes that a control
// does not write, or whose source lane is outside the row, receive `ident`.
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v, uint32_t ident) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
      static_cast<int>(ident), static_cast<int>(v), CTRL, ROWS, 0xf, false));
}

// v of lane (lane ^ j) for j in {1, 2, 4, 8, 16, 32}, inside the VALU:
// quad_perm for 1 and 2, row_shl:4 / row_shr:4 restricted to alternate banks
// of 4 lanes for 4, row_ror:8 for 8, and the gfx950 lane swaps for 16 and 32
// (permlane16_swap exchanges rows 0<->1 and 2<->3, permlane32_swap the two
// halves; of the pair returned for (v, v), element 0 holds the partner value
// in the upper row / half and element 1 in the lower).  j is a compile-time
// constant after unrolling at every call site.  The controls for 1, 2 and 8
// write every lane from a lane of the same row, so their moves need no prior
// value (mov_dpp: no copy of v into the destination first); for 4 the first
// move's unwritten banks are written by the second.
__device__ __forceinline__ uint32_t lane_xor_u32(uint32_t v, int j) {
  const int x = static_cast<int>(v);
  switch (j) {
  case 1:
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(x, 0xB1, 0xf, 0xf, false));
  case 2:
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(x, 0x4E, 0xf, 0xf, false));
  case 4: {
    const int t = __builtin_amdgcn_mov_dpp(x, 0x104, 0xf, 0x5, false);
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(t, x, 0x114, 0xf, 0xA, false));
  }
  case 8:
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(x, 0x128, 0xf, 0xf, false));
  case 16: {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (__lane_id() & 16) ? r[0] : r[1];
  }
  default: {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (__lane_id() & 32) ? r[0] : r[1];
  }
  }
}
__device__ __forceinline__ int32_t lane_xor_i32(int32_t v, int j) {
  return static_cast<int32_t>(lane_xor_u32(static_cast<uint32_t>(v), j));
}
__device__ __forceinline__ float lane_xor_f32(float v, int j) {
  return __uint_as_float(lane_xor_u32(__float_as_uint(v), j));
}

// Minimum / maximum over the wave, returned wave-uniform.
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  constexpr uint32_t I = 0xFFFFFFFFu;
  v = min(v, dpp_u32<0xB1>(v, I));
  v = min(v, dpp_u32<0x4E>(v, I));
  v = min(v, dpp_u32<0x141>(v, I));
  v = min(v, dpp_u32<0x140>(v, I));
  v = min(v, dpp_u32<0x142, 0xa>(v, I));
  v = min(v, dpp_u32<0x143, 0xc>(v, I));
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v, 0u));
  v = max(v, dpp_u32<0x4E>(v, 0u));
  v = max(v, dpp_u32<0x141>(v, 0u));
  v = max(v, dpp_u32<0x140>(v, 0u));
  v = max(v, dpp_u32<0x142, 0xa>(v, 0u));
  v = max(v, dpp_u32<0x143, 0xc>(v, 0u));
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}

// Inclusive prefix sum across the 64 lanes: Kogge-Stone inside each row of 16
// (row_shr 1, 2, 4, 8), then the row totals carried by the two broadcasts.
__device__ __forceinline__ int32_t wave_incl_scan(int32_t v) {
  uint32_t u = static_cast<uint32_t>(v);
  u += dpp_u32<0x111>(u, 0u);
  u += dpp_u32<0x112>(u, 0u);
  u += dpp_u32<0x114>(u, 0u);
  u += dpp_u32<0x118>(u, 0u);
  u += dpp_u32<0x142, 0xa>(u, 0u);
  u += dpp_u32<0x143, 0xc>(u, 0u);
  return static_cast<int32_t>(u);
}

// Inclusive prefix maximum across the 64 lanes (same network as the sum).
__device__ __forceinline__ int32_t wave_incl_max(int32_t v) {
  // Offset by 2^31 so that signed order becomes unsigned order with 0 as the
  // identity.
  uint32_t u = static_cast<uint32_t>(v) ^ 0x80000000u;
  u = max(u, dpp_u32<0x111>(u, 0u));
  u = max(u, dpp_u32<0x112>(u, 0u));
  u = max(u, dpp_u32<0x114>(u, 0u));
  u = max(u, dpp_u32<0x118>(u, 0u));
  u = max(u, dpp_u32<0x142, 0xa>(u, 0u));
  u = max(u, dpp_u32<0x143, 0xc>(u, 0u));
  return static_cast<int32_t>(u ^ 0x80000000u);
}

__device__ __forceinline__ int32_t wave_sum(int32_t v) {
  return __builtin_amdgcn_readlane(wave_incl_scan(v), 63);
}

// Term of nonzero (r, c) in the is_symmetric mirror check: sign(c - r) times
// a multiply-xorshift mix of the packed pair (min, max) (one round of the
// splitmix64 finalizer of Steele, Lea and Flood, OOPSLA 2014), 0 on the
// diagonal.  Summed mod 2^64 over a pattern that is symmetric as a multiset,
// the terms cancel exactly; an asymmetric one leaves
// (count(a, b) - count(b, a)) * H(a, b) terms, which cancel only when its
// unmatched pairs' mixes happen to sum to zero mod 2^64.
__device__ __forceinline__ uint64_t mirror_term(int32_t r, int32_t c) {
  if (r == c) return 0;
  const uint32_t a = static_cast<uint32_t>(r < c ? r : c), b = static_cast<uint32_t>(r < c ? c : r);
  uint64_t x = ((static_cast<uint64_t>(a) << 32) | b) ^ 0x9e3779b97f4a7c15ull;
  x = (x ^ (x >> 31)) * 0xbf58476d1ce4e5b9ull;
  x ^= x >> 29;
  return c > r ? x : 0ull - x;
}

// weighted_index packing (reference sporder/src/common/weighted_index.h:15-27).
__device__ __forceinline__ uint64_t pack_wi(int32_t index, float weight) {
  return (static_cast<uint64_t>(__float_as_uint(weight)) << 32) |
         static_cast<uint32_t>(index + 1);
}
__device__ __forceinline__ int32_t wi_index(uint64_t v) {
  return static_cast<int32_t>(static_cast<uint32_t>(v)) - 1;
}
__device__ __forceinline__ float wi_weight(uint64_t v) {
  return __uint_as_float(static_cast<uint32_t>(v >> 32));
}

} // namespace sporder_hip

struct sporder_context_struct {
  sporder_hip::Context impl;
};
