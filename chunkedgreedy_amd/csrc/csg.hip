// csg.hip -- Chunked Greedy (sporder-csg): table construction, the
// per-chunk greedy chain, table statistics, and the C-ABI entry points
// sporder_chunk_similarity_greedy, sporder_similarity_graph and
// sporder_chunk_similarity_top_k.
//
// Semantics follow the reference bit for bit:
//   sketch stream  sporder/src/common/chunk_similarity_top_k.cu:30-88
//   space-saving   sporder/src/common/warp_spacesaving.cuh:12-151 (sketch.hpp)
//   greedy         sporder/src/csg/chunk_similarity_greedy.cu:14-98
//   stats          sporder/src/common/similarity_top_k.cu:120-172,
//                  sporder/src/csg/stats_collector.cu:43-63
//
// Table construction picks, per call:
//   - chunk-local (csg_local.hip): one workgroup per chunk, transpose in LDS,
//     when chunk_size <= kLocalRowCap and the packed keys fit 32 bits; chunks
//     with more nonzeros than LDS holds overflow to
//   - global-CSC (csg_overflow.hip): the reference's access pattern
//     (transpose, or the CSR itself when is_symmetric); each nonzero's run of
//     chunk rows in its column is found by a device-wide pass, then one wave
//     per row streams the runs into the sketch.
// Both produce the same table.
//
// Greedy: one wave per chunk.  For chunk_size <= kGreedyCompactRows (with at
// most 2^20 table entries per chunk) the chunk's in-chunk table entries are
// compacted into LDS (per-row offsets,
// each row sorted into the chain's preference order, offsets turned into row
// headers that carry the first entry) so the serial chain touches only LDS;
// slices past the LDS capacity, and longer chunks, read the table in global
// memory.  With many chunks the sketch also writes per-row valid counts, and
// sparse slices are staged from them row by row.
#include "common.hpp"
#include "sketch.hpp"

#include <algorithm>
#include <chrono>
#include <cstring>
#include <type_traits>

namespace sporder_hip {

namespace {

// ---- greedy chain ----------------------------------------------------------

struct ChainCounters {
  int32_t restarts;
  int32_t links;
  double link_weight_sum;
  double in_chunk_weight; // weight of table entries inside their row's chunk
};

// The visited bitmap of a chain is written by every lane of the wave with the
// same value (each lane ORs the same bit into the same word), so each lane's
// own program order makes its later reads see every update: no cross-lane
// fence is needed inside the chain loop.
__device__ __forceinline__ void mark_visited(uint32_t *bm, int32_t b) {
  bm[b >> 5] |= 1u << (b & 31);
}

// Lowest unvisited bit at or after word *low_word; advances *low_word (the
// lowest unvisited row never moves backwards).  Returns -1 when none is left.
__device__ __forceinline__ int32_t next_unvisited(const uint32_t *bm, int32_t words,
                                                  uint32_t tail_mask, int32_t *low_word) {
  const int lane = lane_id();
  while (*low_word < words) {
    int32_t w = *low_word + lane;
    uint32_t free_bits = 0u;
    if (w < words) free_bits = ~bm[w] & (w == words - 1 ? tail_mask : 0xFFFFFFFFu);
    uint64_t m = ballot(free_bits != 0u);
    if (m) {
      int first = __builtin_ctzll(m);
      uint32_t fb = static_cast<uint32_t>(readlane(static_cast<int32_t>(free_bits), first));
      *low_word += first;
      return *low_word * 32 + __builtin_ctz(fb);
    }
    *low_word += kWave;
  }
  return -1;
}

// Best (max weight, ties -> smaller index) over the wave; all lanes get it.
// A lane offers a candidate when *c >= 0; candidate weights are table weights,
// which are positive, so their bit patterns order like the values.  With no
// candidate anywhere the result is (-1.0f, -1).
__device__ __forceinline__ void wave_argmax(float *w, int32_t *c) {
  const uint32_t wb = *c >= 0 ? __float_as_uint(*w) : 0u;
  const uint32_t wmax = wave_max_u32(wb);
  if (wmax == 0u) {
    *w = -1.0f;
    *c = -1;
    return;
  }
  const uint32_t cmin =
      wave_min_u32((*c >= 0 && wb == wmax) ? static_cast<uint32_t>(*c) : 0xFFFFFFFFu);
  *w = __uint_as_float(wmax);
  *c = static_cast<int32_t>(cmin);
}

constexpr int kGreedyBlock = 256;
constexpr int kGreedyWaves = kGreedyBlock / kWave;

// General greedy: one wave per chunk, table rows read from global memory.
// `words_per_wave` u32 words of visited bitmap per wave live in LDS (use_lds)
// or in `gbitmap` at chunk * words_per_wave.
__global__ void __launch_bounds__(kGreedyBlock)
    greedy_kernel(int32_t n, int32_t k, int32_t chunk_size, int32_t num_chunks,
                  const uint64_t *__restrict__ table, int32_t *__restrict__ order,
                  ChainCounters *counters, uint32_t *gbitmap,
                  int32_t words_per_wave, int use_lds) {
  extern __shared__ uint32_t lds_bitmap[];
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int64_t chunk = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + wave;
  if (chunk >= num_chunks) return;
  const int64_t start64 = chunk * chunk_size;
  const int32_t start = static_cast<int32_t>(start64);
  const int32_t end =
      static_cast<int32_t>(start64 + chunk_size > n ? n : start64 + chunk_size);
  if (start >= end) return;
  const int32_t size = end - start;
  const int32_t words = (size + 31) >> 5;
  uint32_t *bm = use_lds ? lds_bitmap + static_cast<size_t>(wave) * words_per_wave
                         : gbitmap + static_cast<size_t>(chunk) * words_per_wave;
  // Every lane clears every word, so each lane's later reads follow its own
  // writes (see mark_visited).
  for (int32_t w = 0; w < words; ++w) bm[w] = 0u;

  const uint32_t tail_mask = (size & 31) ? ((1u << (size & 31)) - 1u) : 0xFFFFFFFFu;
  int32_t cur = start, pos = start, low_word = 0;
  int32_t restarts = 0, links = 0;
  float link_w = 0.0f;
  double in_w = 0.0; // per lane

  // One position of [start, end) per step; the bound only ends a walk whose
  // bitmap went wrong before it could write past its chunk.
  while (pos < end) {
    mark_visited(bm, cur - start);
    if (!use_lds) {
      // Global-memory bitmap: order the store before the loads that test it.
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    }
    if (lane == 0) order[pos] = cur;
    pos += 1;

    const uint64_t *row = table + static_cast<size_t>(cur) * k;
    float best_w = -1.0f;
    int32_t best_c = -1;
    for (int32_t j = lane; j < k; j += kWave) {
      uint64_t e = row[j];
      int32_t cand = wi_index(e);
      if (cand < 0) break; // valid entries form a prefix
      if (cand < start || cand >= end) continue;
      in_w += wi_weight(e);
      int32_t b = cand - start;
      if (bm[b >> 5] & (1u << (b & 31))) continue;
      float w = wi_weight(e);
      if (w > best_w || (w == best_w && cand < best_c)) {
        best_w = w;
        best_c = cand;
      }
    }
    wave_argmax(&best_w, &best_c);
    best_c = __builtin_amdgcn_readfirstlane(best_c);
    if (best_c >= 0) {
      links += 1;
      link_w += readlane_f(best_w, 0);
      cur = best_c;
      continue;
    }
    int32_t nxt = next_unvisited(bm, words, tail_mask, &low_word);
    if (nxt < 0) break;
    restarts += 1;
    cur = start + nxt;
  }
  if (counters != nullptr) {
    if (in_w != 0.0) atomicAdd(&counters->in_chunk_weight, in_w);
    if (lane == 0) {
      atomicAdd(&counters->restarts, restarts);
      atomicAdd(&counters->links, links);
      atomicAdd(&counters->link_weight_sum, static_cast<double>(link_w));
    }
  }
}

// Compact greedy: chunks of at most kGreedyCompactRows rows.  Four waves
// count each row's valid entries that fall inside the chunk (the only ones the
// chain can follow; all of them for a chunk-restricted table, a few for the
// global one) and stage them, unordered, in LDS; the counts are scanned into
// per-row offsets and the staged entries moved to their rows as
// (weight bits << 32 | local index); then wave 0 runs the chain on LDS alone.
// The table slice is read once.  A slice with more than `entry_cap` in-chunk
// entries keeps the offsets in LDS and reads the rows from global memory.
constexpr int kGreedyCompactRows = 4096;

// Walk modes of greedy_compact_kernel.
constexpr int kWalkTable = 0, kWalkSingle = 1, kWalkAhead = 2;
// Packed rows (no statistics): a slice of up to kPackedCap in-chunk entries
// whose rows have at most kPackedMaxK table entries is held as 16-bit local
// indices in preference order; the walk needs no weights.
constexpr int32_t kPackedCap = 16384;
constexpr int32_t kPackedMaxK = 32;
// Compacted rows: the offsets array becomes row headers, the offset in the low
// kOffBits bits (at most 32 * kGreedyBlock entries, or kPackedCap packed ones)
// and the local index of the row's first (preferred) entry above it (below
// kGreedyCompactRows).
constexpr int kOffBits = 15;
constexpr int32_t kOffMask = (1 << kOffBits) - 1;
static_assert(32 * kGreedyBlock <= kOffMask && kPackedCap <= kOffMask &&
                  kGreedyCompactRows <= 4096 && kOffBits + 12 <= 31,
              "row header fields");

// Byte offset of a pointer into this workgroup's LDS (for LDS instructions
// written in assembly).
__device__ __forceinline__ uint32_t lds_offset(const void *p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void *)(p)));
}

// Why ahead_steps returned.
constexpr int32_t kStepsEnd = 0;     // pos reached end
constexpr int32_t kStepsRestart = 1; // cur placed; its row has no free in-chunk entry
constexpr int32_t kStepsLong = 2;    // cur placed; its row has more than 64 entries
constexpr int32_t kStepsRing = 3;    // 64 positions in the ring; cur not yet placed

// Steps of the read-ahead walk (compacted rows in LDS, at most 64 bitmap
// words), written as one block of GCN assembly; the compiled step issues about
// a hundred instructions, most of them on the branch structure around its
// three LDS reads.  One step: mark cur in the visited bitmap (lane w holds
// word w), record start + cur in slot rp of the position ring, then take the
// row's entries [d0, d1) (one per lane, lanes past the row repeat its last
// one), read each entry's row headers s_off[c], s_off[c + 1] and its visited
// bit (a ds_bpermute of the bitmap word), and move to the first entry that
// is free -- the row's preference order -- with its headers as the next
// row's.  Runs while pos < end and the ring has room; returns at the first
// row that has no free entry or more than 64 entries (the caller finishes
// that step), with nd0, nd1 the headers of the row last placed.  The ring's
// rp slots (positions pos - rp ..) are the caller's to store.  With 64-bit
// entries the chosen entry's weight is added to link_w and links counted as
// the compiled step does.
//
// Wait states: a VALU write of an SGPR is read by a VALU instruction at least
// two instructions later (v_readlane of the weight, then s_nop 1); lane selects
// of v_readlane are written by s_ff1 three scalar instructions before.  LDS
// instructions need no M0 here.  Every lane of the wave must be active.
template <bool kPacked>
__device__ __forceinline__ int32_t ahead_steps(uint32_t &bm0, uint32_t &ring, int32_t &rp,
                                               int32_t &cur, int32_t &nd0, int32_t &nd1,
                                               int32_t &pos, int32_t &links, float &link_w,
                                               int32_t end, int32_t start, int32_t lane,
                                               uint32_t ent_lds, uint32_t off_lds) {
  int32_t st, w, d0, d1, len, lm1, l, wl;
  uint64_t m, lm;
  uint32_t vt, vval, vj, va, vcl, vwt, vo, vo0, vo1, vw, vword;
  // All wave-uniform; readfirstlane states it, so that the compiler hands
  // them over in scalar registers.
  cur = __builtin_amdgcn_readfirstlane(cur);
  nd0 = __builtin_amdgcn_readfirstlane(nd0);
  nd1 = __builtin_amdgcn_readfirstlane(nd1);
  pos = __builtin_amdgcn_readfirstlane(pos);
  links = __builtin_amdgcn_readfirstlane(links);
  rp = __builtin_amdgcn_readfirstlane(rp);
  end = __builtin_amdgcn_readfirstlane(end);
  ent_lds = __builtin_amdgcn_readfirstlane(ent_lds);
  off_lds = __builtin_amdgcn_readfirstlane(off_lds);
  asm volatile(
      "0:\n\t"
      "s_cmp_ge_i32 %[pos], %[end]\n\t"
      "s_cbranch_scc1 8f\n\t"
      "s_cmp_eq_u32 %[rp], 64\n\t"
      "s_cbranch_scc1 5f\n\t"
      // mark cur: word cur >> 5 (lane), bit cur & 31
      "s_lshr_b32 %[w], %[cur], 5\n\t"
      "v_cmp_eq_u32_e32 vcc, %[w], %[lane]\n\t"
      "v_lshlrev_b32_e64 %[vt], %[cur], 1\n\t"
      "v_cndmask_b32_e32 %[vt], 0, %[vt], vcc\n\t"
      "v_or_b32_e32 %[bm0], %[bm0], %[vt]\n\t"
      // ring slot rp <- start + cur
      "v_cmp_eq_u32_e32 vcc, %[rp], %[lane]\n\t"
      "v_add_u32_e32 %[vval], %[cur], %[startv]\n\t"
      "v_cndmask_b32_e32 %[ring], %[ring], %[vval], vcc\n\t"
      "s_add_u32 %[rp], %[rp], 1\n\t"
      "s_add_u32 %[pos], %[pos], 1\n\t"
      // cur's entries [d0, d1)
      "s_and_b32 %[d0], %[nd0], 0x7fff\n\t"
      "s_and_b32 %[d1], %[nd1], 0x7fff\n\t"
      "s_sub_i32 %[len], %[d1], %[d0]\n\t"
      "s_cmp_lt_i32 %[len], 1\n\t"
      "s_cbranch_scc1 7f\n\t"
      "s_cmp_gt_i32 %[len], 64\n\t"
      "s_cbranch_scc1 6f\n\t"
      "s_sub_u32 %[lm1], %[len], 1\n\t"
      "v_min_u32_e32 %[vj], %[lm1], %[lane]\n\t"
      "v_add_u32_e32 %[vj], %[d0], %[vj]\n\t"
      ".if %[packed]\n\t"
      "v_lshl_add_u32 %[va], %[vj], 1, %[entl]\n\t"
      "ds_read_u16 %[vcl], %[va]\n\t"
      ".else\n\t"
      "v_lshl_add_u32 %[va], %[vj], 3, %[entl]\n\t"
      "ds_read_b32 %[vcl], %[va]\n\t"
      "ds_read_b32 %[vwt], %[va] offset:4\n\t"
      ".endif\n\t"
      "v_cmp_gt_u32_e64 %[lm], %[len], %[lane]\n\t"
      "s_waitcnt lgkmcnt(0)\n\t"
      // each entry's row headers and visited bit
      "v_lshl_add_u32 %[vo], %[vcl], 2, %[offl]\n\t"
      "ds_read_b32 %[vo0], %[vo]\n\t"
      "ds_read_b32 %[vo1], %[vo] offset:4\n\t"
      "v_lshrrev_b32_e32 %[vw], 3, %[vcl]\n\t"
      "ds_bpermute_b32 %[vword], %[vw], %[bm0]\n\t"
      "s_waitcnt lgkmcnt(0)\n\t"
      "v_lshrrev_b32_e32 %[vword], %[vcl], %[vword]\n\t"
      "v_and_b32_e32 %[vword], 1, %[vword]\n\t"
      "v_cndmask_b32_e64 %[vword], 1, %[vword], %[lm]\n\t"
      "v_cmp_eq_u32_e64 %[m], 0, %[vword]\n\t"
      "s_ff1_i32_b64 %[l], %[m]\n\t"
      "s_cmp_lt_i32 %[l], 0\n\t"
      "s_cbranch_scc1 7f\n\t"
      "s_add_u32 %[links], %[links], 1\n\t"
      "v_readlane_b32 %[cur], %[vcl], %[l]\n\t"
      "v_readlane_b32 %[nd0], %[vo0], %[l]\n\t"
      "v_readlane_b32 %[nd1], %[vo1], %[l]\n\t"
      ".if %[packed] == 0\n\t"
      "v_readlane_b32 %[wl], %[vwt], %[l]\n\t"
      "s_nop 1\n\t"
      "v_add_f32_e32 %[linkw], %[wl], %[linkw]\n\t"
      ".endif\n\t"
      "s_branch 0b\n"
      "5:\n\t"
      "s_mov_b32 %[st], 3\n\t"
      "s_branch 9f\n"
      "6:\n\t"
      "s_mov_b32 %[st], 2\n\t"
      "s_branch 9f\n"
      "7:\n\t"
      "s_mov_b32 %[st], 1\n\t"
      "s_branch 9f\n"
      "8:\n\t"
      "s_mov_b32 %[st], 0\n"
      "9:"
      : [bm0] "+v"(bm0), [ring] "+v"(ring), [linkw] "+v"(link_w), [rp] "+s"(rp),
        [cur] "+s"(cur), [nd0] "+s"(nd0), [nd1] "+s"(nd1), [pos] "+s"(pos),
        [links] "+s"(links), [st] "=&s"(st), [w] "=&s"(w), [d0] "=&s"(d0), [d1] "=&s"(d1),
        [len] "=&s"(len), [lm1] "=&s"(lm1), [l] "=&s"(l), [wl] "=&s"(wl), [m] "=&s"(m),
        [lm] "=&s"(lm), [vt] "=&v"(vt), [vval] "=&v"(vval), [vj] "=&v"(vj), [va] "=&v"(va),
        [vcl] "=&v"(vcl), [vwt] "=&v"(vwt), [vo] "=&v"(vo), [vo0] "=&v"(vo0),
        [vo1] "=&v"(vo1), [vw] "=&v"(vw), [vword] "=&v"(vword)
      : [end] "s"(end), [startv] "v"(start), [lane] "v"(lane), [entl] "s"(ent_lds),
        [offl] "s"(off_lds), [packed] "i"(kPacked ? 1 : 0)
      : "vcc", "scc", "memory");
  return st;
}

// The walk's restart for chunks of at most 64 bitmap words, as one block of
// GCN assembly (the compiled search issues about 65 instructions per bitmap
// word).  Per word, lowest first from low_word: the word's free rows (lane w
// of ~bm0, masked by full_lane: the chunk's rows of that word, 0 past the
// chunk's words); the rows among them that have entries (headers s_off[r],
// s_off[r + 1], read by every lane for row min(w * 32 + (lane & 31), size - 1));
// the free rows below the first row with entries are emitted in index order at
// positions pos .. (stored while below end_rel, relative to the chunk's
// order_chunk), marked visited and counted into pos and restarts.  Returns the
// first free row with entries (the walk continues there), or -1 when no row
// is free.  kSorted: headers carry the first entry above kOffBits.  The block
// stores the emitted rows itself, under an exec mask of those lanes (the entry
// mask is restored after the store); every lane of the wave must be active.
template <bool kSorted>
__device__ __forceinline__ int32_t restart_search(uint32_t &bm0, int32_t &low_word,
                                                  int32_t &pos, int32_t &restarts,
                                                  int32_t lane, uint32_t full_lane,
                                                  uint32_t off_lds, int32_t size_m1,
                                                  int32_t *order_chunk, int32_t start,
                                                  int32_t end_rel) {
  int32_t nxt, w, rb, fb, we, fe, em, emx, prel, sr, c;
  uint64_t m, sx;
  uint32_t vf, vr, va, vo0, vo1, vi, vval, vt, vl31;
  low_word = __builtin_amdgcn_readfirstlane(low_word);
  pos = __builtin_amdgcn_readfirstlane(pos);
  restarts = __builtin_amdgcn_readfirstlane(restarts);
  off_lds = __builtin_amdgcn_readfirstlane(off_lds);
  size_m1 = __builtin_amdgcn_readfirstlane(size_m1);
  start = __builtin_amdgcn_readfirstlane(start);
  end_rel = __builtin_amdgcn_readfirstlane(end_rel);
  const uint64_t obase = static_cast<uint64_t>(reinterpret_cast<uintptr_t>(order_chunk));
  const uint64_t ob = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(
                          static_cast<int32_t>(obase))) |
                      (static_cast<uint64_t>(static_cast<uint32_t>(
                           __builtin_amdgcn_readfirstlane(static_cast<int32_t>(obase >> 32))))
                       << 32);
  asm volatile(
      "s_mov_b32 %[nxt], -1\n\t"
      "v_and_b32_e32 %[vl31], 31, %[lane]\n"
      "1:\n\t"
      // lowest word at or after low_word with a free row
      "v_not_b32_e32 %[vf], %[bm0]\n\t"
      "v_and_b32_e32 %[vf], %[vf], %[full]\n\t"
      "v_cmp_le_u32_e32 vcc, %[low], %[lane]\n\t"
      "v_cndmask_b32_e32 %[vf], 0, %[vf], vcc\n\t"
      "v_cmp_ne_u32_e64 %[m], 0, %[vf]\n\t"
      "s_ff1_i32_b64 %[w], %[m]\n\t"
      "s_cmp_lt_i32 %[w], 0\n\t"
      "s_cbranch_scc1 9f\n\t"
      "s_mov_b32 %[low], %[w]\n\t"
      "s_lshl_b32 %[rb], %[w], 5\n\t"
      "v_readlane_b32 %[fb], %[vf], %[w]\n\t"
      // which of the word's rows have entries
      "v_add_u32_e32 %[vr], %[rb], %[vl31]\n\t"
      "v_min_u32_e32 %[vr], %[szm1], %[vr]\n\t"
      "v_lshl_add_u32 %[va], %[vr], 2, %[offl]\n\t"
      "ds_read_b32 %[vo0], %[va]\n\t"
      "ds_read_b32 %[vo1], %[va] offset:4\n\t"
      "s_waitcnt lgkmcnt(0)\n\t"
      ".if %[sorted]\n\t"
      "v_and_b32_e32 %[vo0], 0x7fff, %[vo0]\n\t"
      "v_and_b32_e32 %[vo1], 0x7fff, %[vo1]\n\t"
      ".endif\n\t"
      "v_cmp_gt_u32_e32 vcc, %[vo1], %[vo0]\n\t"
      "s_and_b32 %[we], vcc_lo, %[fb]\n\t"
      // emit = we ? fb & ((1 << ctz(we)) - 1) : fb
      "s_ff1_i32_b32 %[fe], %[we]\n\t"
      "s_bfm_b32 %[em], %[fe], 0\n\t"
      "s_and_b32 %[em], %[em], %[fb]\n\t"
      "s_cmp_eq_u32 %[we], 0\n\t"
      "s_cselect_b32 %[em], %[fb], %[em]\n\t"
      "s_cmp_eq_u32 %[em], 0\n\t"
      "s_cbranch_scc1 3f\n\t"
      // store the emitted rows at pos + their rank, below end
      "s_sub_u32 %[prel], %[pos], %[start]\n\t"
      "v_mbcnt_lo_u32_b32 %[vi], %[em], 0\n\t"
      "v_add_u32_e32 %[vi], %[prel], %[vi]\n\t"
      "v_cmp_gt_u32_e32 vcc, %[endrel], %[vi]\n\t"
      "s_and_b32 %[emx], vcc_lo, %[em]\n\t"
      "s_add_u32 %[sr], %[rb], %[start]\n\t"
      "v_add_u32_e32 %[vval], %[sr], %[vl31]\n\t"
      "v_lshlrev_b32_e32 %[vi], 2, %[vi]\n\t"
      "s_mov_b64 %[sx], exec\n\t"
      "s_mov_b32 exec_hi, 0\n\t"
      "s_mov_b32 exec_lo, %[emx]\n\t"
      "global_store_dword %[vi], %[vval], %[ob]\n\t"
      "s_mov_b64 exec, %[sx]\n\t"
      // mark them visited
      "v_cmp_eq_u32_e32 vcc, %[w], %[lane]\n\t"
      "v_mov_b32_e32 %[vt], %[em]\n\t"
      "v_cndmask_b32_e32 %[vt], 0, %[vt], vcc\n\t"
      "v_or_b32_e32 %[bm0], %[bm0], %[vt]\n\t"
      "s_bcnt1_i32_b32 %[c], %[em]\n\t"
      "s_add_u32 %[pos], %[pos], %[c]\n\t"
      "s_add_u32 %[rst], %[rst], %[c]\n"
      "3:\n\t"
      "s_cmp_eq_u32 %[we], 0\n\t"
      "s_cbranch_scc1 1b\n\t"
      "s_add_u32 %[nxt], %[rb], %[fe]\n"
      "9:"
      : [bm0] "+v"(bm0), [low] "+s"(low_word), [pos] "+s"(pos), [rst] "+s"(restarts),
        [nxt] "=&s"(nxt), [w] "=&s"(w), [rb] "=&s"(rb), [fb] "=&s"(fb), [we] "=&s"(we),
        [fe] "=&s"(fe), [em] "=&s"(em), [emx] "=&s"(emx), [prel] "=&s"(prel), [sr] "=&s"(sr),
        [c] "=&s"(c), [m] "=&s"(m), [sx] "=&s"(sx), [vf] "=&v"(vf), [vr] "=&v"(vr), [va] "=&v"(va),
        [vo0] "=&v"(vo0), [vo1] "=&v"(vo1), [vi] "=&v"(vi), [vval] "=&v"(vval), [vt] "=&v"(vt),
        [vl31] "=&v"(vl31)
      : [lane] "v"(lane), [full] "v"(full_lane), [offl] "s"(off_lds), [szm1] "s"(size_m1),
        [ob] "s"(ob), [start] "s"(start), [endrel] "s"(end_rel), [sorted] "i"(kSorted ? 1 : 0)
      : "vcc", "scc", "memory");
  return nxt;
}

// Rows of at most kPackedSortK table entries are packed by a sorting network
// in registers (pack_row_sorted).
constexpr int32_t kPackedSortK = 16;

// The in-chunk entries of a row's valid prefix (rv <= kPackedSortK) in
// preference order, written to out[0 ..): table order is weight descending,
// so each run of equal weight (numbered in table order) is put in local-index
// order, as keys (run << 16) | local sorted ascending; entries outside the
// chunk sort last.  Returns how many were written.
__device__ __forceinline__ int32_t pack_row_sorted(const uint64_t *__restrict__ row, int32_t rv,
                                                   int32_t start, int32_t end, uint16_t *out) {
  constexpr int KM = kPackedSortK;
  uint32_t key[KM];
  int32_t cnt = 0;
  uint32_t run = 0u, prev_w = 0u; // weights are positive: 0 matches none
#pragma unroll
  for (int j = 0; j < KM; ++j) {
    const uint64_t e = j < rv ? row[j] : 0ull;
    const int32_t c = wi_index(e);
    const bool in = j < rv && c >= start && c < end;
    const uint32_t wb = static_cast<uint32_t>(e >> 32);
    run += (in && wb != prev_w) ? 1u : 0u;
    prev_w = in ? wb : prev_w;
    key[j] = in ? ((run << 16) | static_cast<uint32_t>(c - start)) : 0xFFFFFFFFu;
    cnt += in ? 1 : 0;
  }
#pragma unroll
  for (int kk = 2; kk <= KM; kk <<= 1) {
#pragma unroll
    for (int jj = kk >> 1; jj > 0; jj >>= 1) {
#pragma unroll
      for (int i = 0; i < KM; ++i) {
        const int l = i ^ jj;
        if (l > i) {
          const uint32_t x = key[i], y = key[l];
          const bool swap = ((i & kk) == 0) ? (x > y) : (x < y);
          key[i] = swap ? y : x;
          key[l] = swap ? x : y;
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < KM; ++j) {
    if (j < cnt) out[j] = static_cast<uint16_t>(key[j] & 0xFFFFu);
  }
  return cnt;
}

// 64-bit words of the entries region: entry_cap staged entries, or packed_cap
// 16-bit ones in the same bytes.
__host__ __device__ inline int32_t greedy_entry_words(int32_t entry_cap, int32_t packed_cap) {
  return entry_cap > (packed_cap + 3) / 4 ? entry_cap : (packed_cap + 3) / 4;
}

// Dynamic LDS layout: entries u64[greedy_entry_words] | offsets i32[rows_cap + 1] |
// bitmap u32[ceil(rows_cap / 32)] | valid counts u8[rows_cap].  A staged entry is (weight bits << 32) |
// (slice position << 12) | local index: positions are below 4096 * 256 = 2^20
// and local indices below 4096.
size_t greedy_compact_lds(int32_t rows_cap, int32_t entry_cap, int32_t packed_cap = 0) {
  return static_cast<size_t>(greedy_entry_words(entry_cap, packed_cap)) * 8u +
         static_cast<size_t>(rows_cap + 1) * 4u +
         static_cast<size_t>((rows_cap + 31) / 32) * 4u + static_cast<size_t>(rows_cap);
}

// kStagePer: staged entries each thread moves to their rows (entry_cap is at
// most kStagePer * kGreedyBlock).  packed_cap: 16-bit entries the region holds
// for the packed form (0 when statistics are collected or k > kPackedMaxK).
// With band_hi > band_lo the chain is split over two launches by the slice's
// valid entries S (the sketch's counts, row_valid): the launch with in_band
// set takes the chunks with band_lo < S <= band_hi, the other the rest.
template <int kStagePer>
__global__ void __launch_bounds__(kGreedyBlock)
    greedy_compact_kernel(int32_t n, int32_t k, int32_t chunk_size,
                          const uint64_t *__restrict__ table, int32_t *__restrict__ order,
                          ChainCounters *counters, int32_t rows_cap, int32_t entry_cap,
                          int32_t packed_cap, int32_t band_lo, int32_t band_hi, int32_t in_band,
                          const int32_t *__restrict__ row_valid) {
  extern __shared__ uint64_t smem_u64[];
  __shared__ int32_t s_total;
  __shared__ int32_t s_staged;
  __shared__ int32_t s_valid;
  uint64_t *s_ent = smem_u64;
  uint16_t *s_e16 = reinterpret_cast<uint16_t *>(smem_u64); // the packed form
  int32_t *s_off =
      reinterpret_cast<int32_t *>(smem_u64 + greedy_entry_words(entry_cap, packed_cap));
  uint32_t *s_bm = reinterpret_cast<uint32_t *>(s_off + rows_cap + 1);
  uint8_t *s_rv = reinterpret_cast<uint8_t *>(s_bm + (rows_cap + 31) / 32);

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;
  const int64_t chunk = blockIdx.x;
  const int64_t start64 = chunk * chunk_size;
  const int32_t start = static_cast<int32_t>(start64);
  const int32_t end =
      static_cast<int32_t>(start64 + chunk_size > n ? n : start64 + chunk_size);
  const int32_t size = end - start;
  const int32_t words = (size + 31) >> 5;
  const uint64_t *slice = table + static_cast<size_t>(start) * k;
  const int64_t slice_len = static_cast<int64_t>(size) * k;

  for (int32_t r = tid; r <= size; r += kGreedyBlock) s_off[r] = 0;
  for (int32_t w = tid; w < words; w += kGreedyBlock) s_bm[w] = 0u;
  // The sketch's per-row valid counts (k <= 255), when given, and their sum.
  if (tid == 0) {
    s_staged = 0;
    s_valid = 0;
  }
  __syncthreads();
  if (row_valid != nullptr) {
    int32_t vsum = 0;
    for (int32_t r = tid; r < size; r += kGreedyBlock) {
      const int32_t c = min(max(row_valid[start + r], 0), k);
      s_rv[r] = static_cast<uint8_t>(c);
      vsum += c;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) vsum += __shfl_xor(vsum, off, kWave);
    if (lane == 0 && vsum != 0) atomicAdd(&s_valid, vsum);
  }
  __syncthreads();
  if (band_hi > band_lo && row_valid != nullptr &&
      (band_lo < s_valid && s_valid <= band_hi) != (in_band != 0)) {
    return; // the other launch's chunk (uniform across the workgroup)
  }
  // A slice with under a quarter of its entries valid is read row by row, only
  // each row's valid prefix (rows without entries cost no table traffic and a
  // thread waits on one load per row); a denser one is swept whole, coalesced.
  const bool by_rows = row_valid != nullptr && 4 * static_cast<int64_t>(s_valid) < slice_len;
  // Per-row count of valid entries inside the chunk (valid entries form a
  // prefix of each row; only in-chunk entries can be followed), read as a
  // coalesced sweep of the slice.  Rows that also hold out-of-chunk entries
  // (global tables) are flagged in the LDS bitmap; the chain keeps its own
  // visited bitmap in registers.  With counters, the in-chunk weight is summed for the cut
  // statistic.
  double in_w = 0.0;
  if (by_rows) {
    // Same staging as the sweep below, one lane per row: per-lane LDS atomics
    // (few entries), slice positions below 2^20 (checked by the host).
    for (int32_t r = tid; r < size; r += kGreedyBlock) {
      const int32_t rv = s_rv[r];
      const uint64_t *row = slice + static_cast<size_t>(r) * k;
      for (int32_t j0 = 0; j0 < rv; j0 += 4) {
        uint64_t v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = j0 + u < rv ? row[j0 + u] : 0;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int32_t c = wi_index(v[u]); // an empty entry reads as -1
          if (c < 0) continue;
          if (c >= start && c < end) {
            atomicAdd(&s_off[r + 1], 1);
            in_w += wi_weight(v[u]);
            const int32_t si = atomicAdd(&s_staged, 1);
            if (si < entry_cap) {
              s_ent[si] = (v[u] & 0xFFFFFFFF00000000ull) |
                          (static_cast<uint64_t>(r * k + j0 + u) << 12) |
                          static_cast<uint32_t>(c - start);
            }
          } else {
            atomicOr(&s_bm[r >> 5], 1u << (r & 31));
          }
        }
      }
    }
  }
  for (int64_t e0 = static_cast<int64_t>(tid) * 4; !by_rows && e0 < slice_len;
       e0 += static_cast<int64_t>(kGreedyBlock) * 4) {
    uint64_t v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = (e0 + u < slice_len) ? slice[e0 + u] : 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int32_t c = wi_index(v[u]);
      const bool valid = e0 + u < slice_len && c >= 0;
      const bool inside = valid && c >= start && c < end;
      // Staging slots for the wave's in-chunk entries: one LDS atomic per
      // wave, ranks from the ballot.
      const uint64_t m = ballot(inside);
      int32_t base = 0;
      if (m != 0 && lane == 0) base = atomicAdd(&s_staged, __popcll(m));
      base = readlane(base, 0);
      if (valid) {
        const int32_t r = static_cast<int32_t>((e0 + u) / k);
        if (inside) {
          atomicAdd(&s_off[r + 1], 1);
          in_w += wi_weight(v[u]);
          const int32_t si = base + __popcll(m & ((1ull << lane) - 1ull));
          if (si < entry_cap) {
            s_ent[si] = (v[u] & 0xFFFFFFFF00000000ull) |
                        (static_cast<uint64_t>(e0 + u) << 12) |
                        static_cast<uint32_t>(c - start);
          }
        } else {
          atomicOr(&s_bm[r >> 5], 1u << (r & 31));
        }
      }
    }
  }
  if (counters != nullptr) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) in_w += __shfl_xor(in_w, off, kWave);
    if (lane == 0 && in_w != 0.0) atomicAdd(&counters->in_chunk_weight, in_w);
  }
  __syncthreads();
  // Inclusive scan of s_off[1..size] by wave 0 -> offsets.  Wave 0 also
  // counts the rows with exactly one in-chunk entry and those with any.
  int32_t single_rows = 0, entry_rows = 0;
  if (wave == 0) {
    int32_t carry = 0;
    for (int32_t base = 1; base <= size; base += kWave) {
      int32_t i = base + lane;
      int32_t v = i <= size ? s_off[i] : 0;
      single_rows += __popcll(ballot(v == 1));
      entry_rows += __popcll(ballot(v > 0));
      int32_t incl = wave_incl_scan(v) + carry;
      if (i <= size) s_off[i] = incl;
      carry = readlane(incl, kWave - 1);
    }
    if (lane == 0) s_total = carry;
  }
  __syncthreads();
  const int32_t total = s_total;
  const bool compact = total <= entry_cap;
  // Past the staging capacity, rows of at most kPackedMaxK entries are
  // re-read from the slice (now in cache) and packed: each row's in-chunk
  // entries in table order (weight descending), then each run of equal
  // weight sorted by local index, which is the preference order.
  const bool packed = !compact && total <= packed_cap;
  if (packed) {
    for (int32_t r = tid; r < size; r += kGreedyBlock) {
      const int32_t a = s_off[r], b = s_off[r + 1];
      if (b == a) continue;
      const int32_t rv = row_valid != nullptr ? s_rv[r] : k;
      const uint64_t *row = slice + static_cast<size_t>(r) * k;
      if (k <= kPackedSortK) {
        // Rows of at most 16 entries: keys (run number << 16) | local in
        // registers, sorted by a bitonic network with static indices, then
        // stored in order (on a stencil most of a row is one run of equal
        // weight, and the insertion sort below moved nearly every entry).
        const int32_t cnt = pack_row_sorted(row, rv, start, end, s_e16 + a);
        (void)cnt;
        continue;
      }
      uint32_t starts = 0u; // bit t: entry a + t begins a run of equal weight
      uint32_t prev_w = 0u; // weights are positive: 0 matches none
      int32_t o = a;
      for (int32_t j = 0; j < rv && o < b; ++j) {
        const uint64_t e = row[j];
        const int32_t c = wi_index(e);
        if (c < 0) break;
        if (c >= start && c < end) {
          const uint32_t wb = static_cast<uint32_t>(e >> 32);
          if (wb != prev_w) starts |= 1u << (o - a);
          prev_w = wb;
          s_e16[o++] = static_cast<uint16_t>(c - start);
        }
      }
      int32_t rs = a;
      for (int32_t i = a + 1; i < b; ++i) {
        if ((starts >> (i - a)) & 1u) {
          rs = i;
          continue;
        }
        const uint16_t x = s_e16[i];
        int32_t j = i;
        while (j > rs && s_e16[j - 1] > x) {
          s_e16[j] = s_e16[j - 1];
          --j;
        }
        s_e16[j] = x;
      }
    }
    __syncthreads();
    for (int32_t r = tid; r < size; r += kGreedyBlock) {
      const int32_t a = s_off[r], b = s_off[r + 1] & kOffMask;
      if (b > a) s_off[r] = a | (static_cast<int32_t>(s_e16[a]) << kOffBits);
    }
    __syncthreads();
  }
  if (compact) {
    // Entry j of row r moves from its staging slot to s_off[r] + (its rank
    // among the row's in-chunk entries): j itself unless the row is flagged as
    // mixed.  Every thread takes its staged entries into registers before any
    // is overwritten.
    constexpr int kPerThread = kStagePer;
    uint64_t sv[kPerThread];
#pragma unroll
    for (int q = 0; q < kPerThread; ++q) {
      const int32_t i = tid + q * kGreedyBlock;
      sv[q] = i < total ? s_ent[i] : ~0ull;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kPerThread; ++q) {
      if (sv[q] != ~0ull) {
        const uint64_t v = sv[q];
        const int32_t pos = static_cast<int32_t>((v >> 12) & 0xFFFFFu);
        const int32_t local = static_cast<int32_t>(v & 0xFFFu);
        const int32_t r = pos / k, j = pos % k;
        int32_t rank = j;
        if (s_bm[r >> 5] & (1u << (r & 31))) {
          rank = 0;
          const uint64_t *row = slice + static_cast<size_t>(r) * k;
          for (int32_t t = 0; t < j; ++t) {
            const int32_t ct = wi_index(row[t]);
            rank += (ct >= start && ct < end);
          }
        }
        s_ent[s_off[r] + rank] = (v & 0xFFFFFFFF00000000ull) | static_cast<uint32_t>(local);
      }
    }
  }
  __syncthreads();
  if (compact) {
    // Each row's entries into chain preference order: weight descending, then
    // local index ascending.  Entries are (weight bits << 32) | local with
    // positive weights, so with the low word flipped that order is the
    // descending order of the 64-bit value.  Table rows are already in weight
    // order, so the insertion sort only moves entries of equal weight.
    for (int32_t r = tid; r < size; r += kGreedyBlock) {
      const int32_t a = s_off[r], b = s_off[r + 1];
      for (int32_t i = a + 1; i < b; ++i) {
        const uint64_t x = s_ent[i];
        const uint64_t kx = x ^ 0xFFFFFFFFull;
        int32_t j = i;
        while (j > a && (s_ent[j - 1] ^ 0xFFFFFFFFull) < kx) {
          s_ent[j] = s_ent[j - 1];
          --j;
        }
        s_ent[j] = x;
      }
    }
    __syncthreads();
    // Row headers (see kOffBits).  A row's offset bits never change, so reading
    // the next row's offset while its header is written is safe.
    for (int32_t r = tid; r < size; r += kGreedyBlock) {
      const int32_t a = s_off[r], b = s_off[r + 1] & kOffMask;
      if (b > a) s_off[r] = a | (static_cast<int32_t>(s_ent[a] & 0xFFFu) << kOffBits);
    }
    __syncthreads();
  }
  if (wave != 0) return;

  // The chain runs on wave 0 with the visited bitmap in registers: lane l
  // holds words l and 64 + l (chunks of at most kGreedyCompactRows = 4096
  // rows need 128 words).  Cross-lane reads are shuffles issued by every lane
  // (an inactive source lane would read as 0).
  const uint32_t tail_mask = (size & 31) ? ((1u << (size & 31)) - 1u) : 0xFFFFFFFFu;
  uint32_t bm0 = 0u, bm1 = 0u;
  auto full_bits = [&](int32_t w) { return w == words - 1 ? tail_mask : 0xFFFFFFFFu; };
  // Branch-free so that bm0 and bm1 stay registers (a selected reference
  // would turn them into a scratch array).
  auto mark_bits = [&](int32_t w, uint32_t bits) {
    bm0 |= lane == w ? bits : 0u;
    bm1 |= lane + kWave == w ? bits : 0u;
  };
  int32_t cur = 0, pos = start, low_word = 0;
  int32_t restarts = 0, links = 0;
  float link_w = 0.0f;
  // Every step writes one position of [start, end): the bound only ends a
  // walk whose visited bitmap went wrong, before it could write past its
  // chunk.
  // The walk is compiled in three modes (a branch on the mode in every step
  // cost up to 7 % on walks that did not use it):
  //   kWalkTable   slices past the LDS capacity: rows read from the table;
  //   kWalkSingle  compacted, at least half of the rows with entries have
  //                exactly one (mostly one-step links): those take a
  //                lane-read path;
  //   kWalkAhead   compacted, rows of several entries: the next row's offsets
  //                are read during the visited test.
  auto walk = [&](auto mode_tag, auto packed_tag) {
    constexpr int kMode = decltype(mode_tag)::value;
    constexpr bool kPacked = decltype(packed_tag)::value; // 16-bit entries, no weights
    constexpr bool kSorted = kMode != kWalkTable; // rows compacted and sorted in LDS
    constexpr bool kSingle = kMode == kWalkSingle;
    constexpr bool kAhead = kMode == kWalkAhead;
    // Offsets of the next row, read ahead by the step that chose it.
    bool have_next = false;
    int32_t nd0 = 0, nd1 = 0;
    // Read-ahead walks over at most 64 bitmap words run their steps in
    // ahead_steps; a step it hands back (a row without a free entry, or of
    // more than 64 entries) is finished below.
    const bool steps_asm = kAhead && words <= kWave;
    const uint32_t ent_lds = lds_offset(smem_u64), off_lds = lds_offset(s_off);
    // The restart search's rows of each bitmap word (assembly form).
    const uint32_t full_lane = lane < words ? full_bits(lane) : 0u;
    while (pos < end) {
      int32_t steps_st = -1;
      if (kAhead && steps_asm) {
        if (!have_next) {
          nd0 = s_off[cur];
          nd1 = s_off[cur + 1];
        }
        uint32_t ring = 0u;
        int32_t rp = 0;
        steps_st = ahead_steps<kPacked>(bm0, ring, rp, cur, nd0, nd1, pos, links, link_w, end,
                                        start, lane, ent_lds, off_lds);
        if (lane < rp) order[pos - rp + lane] = ring;
        have_next = true; // nd0, nd1: the headers of cur
        if (steps_st == kStepsEnd) break;
        if (steps_st == kStepsRing) continue;
      } else {
        mark_bits(cur >> 5, 1u << (cur & 31));
        if (lane == 0) order[pos] = start + cur;
        pos += 1;
      }
      int32_t h0, h1; // row headers of cur and cur + 1 (offsets for table reads)
      if constexpr (kAhead) {
        h0 = have_next ? nd0 : s_off[cur];
        h1 = have_next ? nd1 : s_off[cur + 1];
        have_next = false;
      } else {
        h0 = s_off[cur];
        h1 = s_off[cur + 1];
      }
      const int32_t d0 = kSorted ? (h0 & kOffMask) : h0;
      const int32_t d1 = kSorted ? (h1 & kOffMask) : h1;
      float best_w = -1.0f;
      int32_t best_c = -1;
      if (d1 > d0 && steps_st != kStepsRestart) {
        // kWalkSingle: the row's first (preferred) entry comes with its header;
        // its visited bit is a lane read of the bitmap word.  Weights are read
        // only for the statistics.  (With read-ahead, taking the first entry
        // this way would give up the next row's early header read: slower on
        // rows of several entries.)
        const int32_t c0 = __builtin_amdgcn_readfirstlane((h0 >> kOffBits) & 0xFFF);
        bool first_free = false;
        if constexpr (kSingle) {
          const int32_t w0 = c0 >> 5;
          const uint32_t word0 =
              static_cast<uint32_t>(w0 < kWave ? readlane(static_cast<int32_t>(bm0), w0)
                                               : readlane(static_cast<int32_t>(bm1), w0 - kWave));
          first_free = c0 < size && !((word0 >> (c0 & 31)) & 1u);
        }
        if (kSingle && (first_free || d1 - d0 == 1)) {
          // The first entry is the step's choice, or the row's only one and
          // visited (most rows that have any on scrambled inputs have one).
          if (first_free) {
            best_c = c0;
            if (!kPacked && counters != nullptr) best_w = wi_weight(s_ent[d0]);
          }
        } else if (kSorted) {
          // The row's in-chunk entries in LDS, in preference order: the step
          // takes the first unvisited one.  With read-ahead, every lane also
          // reads its entry's row offsets while the visited bits are gathered,
          // so the next step starts without an LDS read.  Staged local indices
          // are below `size`, so both reads stay inside the offsets array.
          const int32_t len = d1 - d0;
          for (int32_t j0 = 0; j0 < len && best_c < 0; j0 += kWave) {
            const int32_t j = j0 + lane;
            int32_t cl = -1, o0 = 0, o1 = 0;
            float w = 0.0f;
            if (j < len) {
              if constexpr (kPacked) {
                cl = s_e16[d0 + j];
              } else {
                const uint64_t e = s_ent[d0 + j];
                cl = static_cast<int32_t>(static_cast<uint32_t>(e));
                w = wi_weight(e);
              }
              if constexpr (kAhead) {
                o0 = s_off[cl];
                o1 = s_off[cl + 1];
              }
            }
            const int32_t wi = cl >= 0 ? cl >> 5 : 0;
            uint32_t word =
                static_cast<uint32_t>(__shfl(static_cast<int32_t>(bm0), wi & (kWave - 1), kWave));
            if (words > kWave) { // wave-uniform
              const uint32_t v1 =
                  static_cast<uint32_t>(__shfl(static_cast<int32_t>(bm1), wi & (kWave - 1), kWave));
              word = wi < kWave ? word : v1;
            }
            const uint64_t m = ballot(cl >= 0 && !((word >> (cl & 31)) & 1u));
            if (m != 0) {
              const int l = __builtin_ctzll(m);
              best_c = readlane(cl, l);
              best_w = readlane_f(w, l);
              if constexpr (kAhead) {
                nd0 = readlane(o0, l);
                nd1 = readlane(o1, l);
                have_next = true;
              }
            }
          }
        } else {
          // The row's valid prefix from the table, filtered to the chunk.
          bool open = true; // valid prefix not yet ended
          for (int32_t j0 = 0; j0 < k; j0 += kWave) {
            const int32_t j = j0 + lane;
            int32_t cl = -1;
            float w = 0.0f;
            if (j < k) {
              const uint64_t e = slice[static_cast<size_t>(cur) * k + j];
              const int32_t c = wi_index(e);
              if (c < 0) open = false; // valid entries form a prefix
              cl = (open && c >= start && c < end) ? c - start : -1;
              w = wi_weight(e);
            }
            const int32_t wi = cl >= 0 ? cl >> 5 : 0;
            uint32_t word =
                static_cast<uint32_t>(__shfl(static_cast<int32_t>(bm0), wi & (kWave - 1), kWave));
            if (words > kWave) { // wave-uniform
              const uint32_t v1 =
                  static_cast<uint32_t>(__shfl(static_cast<int32_t>(bm1), wi & (kWave - 1), kWave));
              word = wi < kWave ? word : v1;
            }
            const bool cand = cl >= 0 && !((word >> (cl & 31)) & 1u);
            if (cand && (w > best_w || (w == best_w && cl < best_c))) {
              best_w = w;
              best_c = cl;
            }
            if (ballot(open) != ~0ull) break; // some lane passed the prefix
          }
          const uint64_t m = ballot(best_c >= 0);
          if (m != 0 && (m & (m - 1)) == 0) {
            // One lane holds a candidate: it is the best.
            const int l = __builtin_ctzll(m);
            best_w = readlane_f(best_w, l);
            best_c = readlane(best_c, l);
          } else {
            wave_argmax(&best_w, &best_c);
            best_c = __builtin_amdgcn_readfirstlane(best_c);
          }
        }
      }
      if (best_c >= 0) {
        links += 1;
        link_w += readlane_f(best_w, 0);
        cur = best_c;
        continue;
      }
      // Restart.  The chain now visits the lowest unvisited row; a row with no
      // table entries at all restarts again at once, so the free rows of one
      // bitmap word below the first row that has entries are exactly the next
      // restarts, in index order: emit them in one step.
      int32_t nxt = -1;
      if (words <= kWave) {
        nxt = restart_search<kSorted>(bm0, low_word, pos, restarts, lane, full_lane, off_lds,
                                      size - 1, order + start, start, end - start);
      }
      while (words > kWave) {
        // Lowest word at or after low_word with a free bit.
        const uint32_t f0 =
            (lane < words && lane >= low_word) ? (~bm0 & full_bits(lane)) : 0u;
        const uint32_t f1 = (kWave + lane < words && kWave + lane >= low_word)
                                ? (~bm1 & full_bits(kWave + lane))
                                : 0u;
        const uint64_t m0 = ballot(f0 != 0u), m1 = ballot(f1 != 0u);
        int32_t w = -1;
        uint32_t free_bits = 0u;
        if (m0 != 0) {
          w = __builtin_ctzll(m0);
          free_bits = static_cast<uint32_t>(readlane(static_cast<int32_t>(f0), w));
        } else if (m1 != 0) {
          w = kWave + __builtin_ctzll(m1);
          free_bits = static_cast<uint32_t>(readlane(static_cast<int32_t>(f1), w - kWave));
        }
        if (w < 0) break;
        low_word = w;
        const int32_t r = w * 32 + (lane & 31);
        const bool free_here = lane < 32 && ((free_bits >> (lane & 31)) & 1u);
        const bool has_entries =
            free_here && (kSorted ? (s_off[r + 1] & kOffMask) > (s_off[r] & kOffMask)
                                  : s_off[r + 1] > s_off[r]);
        const uint32_t with_entries = static_cast<uint32_t>(ballot(has_entries));
        const uint32_t emit = with_entries
                                  ? free_bits & ((with_entries & (0u - with_entries)) - 1u)
                                  : free_bits;
        if (emit) {
          if (lane < 32 && ((emit >> lane) & 1u)) {
            // Bounded like the walk itself (a store predicate, not a second
            // exit from this loop).
            const int32_t at = pos + __popc(emit & ((1u << lane) - 1u));
            if (at < end) order[at] = start + r;
          }
          mark_bits(w, emit);
          const int32_t m = __popc(emit);
          pos += m;
          restarts += m;
        }
        if (with_entries) {
          nxt = w * 32 + __builtin_ctz(with_entries);
          break;
        }
      }
      if (nxt < 0) break;
      restarts += 1;
      cur = nxt;
    }
  };
  using Words64 = std::false_type;
  using Words16 = std::true_type;
  if (!compact && !packed) {
    walk(std::integral_constant<int, kWalkTable>{}, Words64{});
  } else if (2 * single_rows >= entry_rows) {
    if (packed) {
      walk(std::integral_constant<int, kWalkSingle>{}, Words16{});
    } else {
      walk(std::integral_constant<int, kWalkSingle>{}, Words64{});
    }
  } else if (packed) {
    walk(std::integral_constant<int, kWalkAhead>{}, Words16{});
  } else {
    walk(std::integral_constant<int, kWalkAhead>{}, Words64{});
  }
  if (counters != nullptr && lane == 0) {
    atomicAdd(&counters->restarts, restarts);
    atomicAdd(&counters->links, links);
    atomicAdd(&counters->link_weight_sum, static_cast<double>(link_w));
  }
}

// ---- table statistics -------------------------------------------------------

// One lane per row.  The row's entries are loaded eight at a time with no
// data-dependent branch between the loads (all k entries of a row exist), so
// the loads of a batch are in flight together; the count and the float sum
// then stop at the first empty entry, as the reference's loop does.  Block
// totals are combined in LDS and added with one atomic per block.
__global__ void __launch_bounds__(256)
    top_k_stats_kernel(int32_t n, int32_t k, const uint64_t *__restrict__ table,
                       TopKTotals *totals) {
  constexpr int kBatch = 8;
  unsigned long long deg_sum = 0;
  double w_sum = 0.0;
  int32_t zeros = 0;
  for (int64_t row = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
       row < n; row += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const uint64_t *r = table + static_cast<size_t>(row) * k;
    int32_t degree = 0;
    float rw = 0.0f;
    bool open = true;
    for (int32_t j0 = 0; j0 < k && open; j0 += kBatch) {
      uint64_t e[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) e[u] = j0 + u < k ? r[j0 + u] : 0ull;
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        open = open && j0 + u < k && wi_index(e[u]) != -1;
        if (open) {
          degree += 1;
          rw += wi_weight(e[u]);
        }
      }
    }
    deg_sum += degree;
    w_sum += rw;
    zeros += (degree == 0);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    deg_sum += __shfl_xor(deg_sum, off, kWave);
    w_sum += __shfl_xor(w_sum, off, kWave);
    zeros += __shfl_xor(zeros, off, kWave);
  }
  __shared__ unsigned long long s_deg[4];
  __shared__ double s_w[4];
  __shared__ int32_t s_zero[4];
  const int wave = threadIdx.x / kWave;
  if (lane_id() == 0) {
    s_deg[wave] = deg_sum;
    s_w[wave] = w_sum;
    s_zero[wave] = zeros;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    deg_sum = s_deg[0] + s_deg[1] + s_deg[2] + s_deg[3];
    w_sum = ((s_w[0] + s_w[1]) + s_w[2]) + s_w[3];
    zeros = s_zero[0] + s_zero[1] + s_zero[2] + s_zero[3];
    if (deg_sum > 0) {
      atomicAdd(&totals->total_degree, deg_sum);
      atomicAdd(&totals->total_weight, w_sum);
    }
    if (zeros > 0) atomicAdd(&totals->zero_degree_rows, zeros);
  }
}

__global__ void unpack_table_kernel(int64_t count, const uint64_t *__restrict__ t,
                                    int32_t *__restrict__ idx,
                                    float *__restrict__ w) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
       i < count; i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    uint64_t e = t[i];
    idx[i] = wi_index(e);
    w[i] = wi_weight(e);
  }
}

void zero_words(Context &ctx, void *p, size_t bytes) {
  fill_u32(ctx, p, static_cast<int64_t>(bytes / 4), 0u);
}

int32_t sketch_m(int32_t k, float oversampling) {
  int32_t m = static_cast<int32_t>(k * oversampling);
  return ((m + 31) / 32) * 32;
}

void validate_sketch_args(int32_t k, float oversampling, int32_t chunk_size) {
  // Reference: sporder/src/common/chunk_similarity_top_k.cu:143-147.
  SP_EXPECT(k > 0, "expect k > 0");
  SP_EXPECT(oversampling >= 1, "expect oversampling >= 1");
  SP_EXPECT(chunk_size >= 1, "expect chunk_size >= 1");
  int32_t m = static_cast<int32_t>(k * oversampling);
  SP_EXPECT(m <= 512, "expect k * oversampling <= 512");
}

// ---- is_symmetric: the CSR read as its own CSC ------------------------------
//
// With is_symmetric the reference takes the CSR as the CSC
// (sporder/src/common/csr2csc.h:49-59): column c's list is row c.  The
// chunk-local sketch transposes each chunk's rows instead.  For input that
// meets the reference's precondition of sorted columns within each row
// (sporder/include/sporder.h:27) the two agree exactly when the pattern is
// symmetric as a multiset (as many (r, c) as (c, r) for every pair).  The
// chunk-local tiers (as they read their rows) and, for the global path's
// rows, a kernel of its own beside that path's sketch add every nonzero's
// mirror_term (common.hpp) into one word; the sum is zero for a symmetric
// pattern.  A call whose sum is not zero is run again
// with every chunk on the global path, which reads the CSR as the CSC like the
// reference.

// A mirror check's device word and whether this call summed into it.
struct MirrorCheck {
  unsigned long long *dev = nullptr;
  bool queued = false;
};

constexpr int kMirrorHostWord = 8; // host_words[8..9] receive the sum

// Queues the copy of the sum; the caller's synchronize makes mirror_failed
// valid.
void mirror_collect(Context &ctx, const MirrorCheck &m) {
  if (!m.queued) return;
  SP_HIP(hipMemcpyAsync(ctx.host_words + kMirrorHostWord, m.dev, sizeof(unsigned long long),
                        hipMemcpyDeviceToHost, ctx.stream));
}

bool mirror_failed(const Context &ctx, const MirrorCheck &m) {
  if (!m.queued) return false;
  unsigned long long sum;
  std::memcpy(&sum, ctx.host_words + kMirrorHostWord, sizeof(sum));
  return sum != 0;
}

// ---- table construction (both paths) ---------------------------------------

size_t table_ws_bytes(int32_t n, int32_t nnz, int32_t k, int32_t chunk_size,
                      bool is_symmetric) {
  size_t b = ws_bytes<uint64_t>(static_cast<size_t>(n) * k);
  int64_t chunks = ceil_div64(n, chunk_size);
  b += ws_bytes<int32_t>(3 * static_cast<size_t>(chunks)) + ws_bytes<int32_t>(4);
  b += chunk_sketch_ws_bytes(n, nnz, chunk_size);
  if (!is_symmetric) {
    b += ws_bytes<int32_t>(static_cast<size_t>(n) + 1) +
         ws_bytes<int32_t>(static_cast<size_t>(nnz)) + csr2csc_ws_bytes(n, nnz);
  } else {
    b += ws_bytes<unsigned long long>(1);
  }
  return b;
}

// Fills `table` (n*k) for the chunked sketch, and `row_valid` (n, when given)
// with each row's number of valid entries.  Records the transpose and
// similarity spans when the spans are enabled.  With `allow_local` false every
// chunk takes the global path.  When is_symmetric chunks go to the chunk-local
// sketch, the sketch kernels sum the mirror check into `mirror`; the caller
// collects it and, if it failed, builds the table again with `allow_local`
// false.
void build_table(Context &ctx, int32_t n, int32_t nnz, const int32_t *d_ptr,
                 const int32_t *d_ind, bool is_symmetric, int32_t k, int32_t m_cap,
                 int32_t chunk_size, uint64_t *table, EventSpan *t_csc,
                 EventSpan *t_sim, MirrorCheck *mirror, bool allow_local,
                 int32_t *row_valid = nullptr) {
  const int64_t chunks = ceil_div64(n, chunk_size);
  int32_t *lists = ctx.take<int32_t>(3 * static_cast<size_t>(chunks));
  int32_t *counts = ctx.take<int32_t>(4);
  const bool local = allow_local && chunk_local_supported(n, chunk_size);
  const bool check_mirror = local && is_symmetric;
  unsigned long long *msum = nullptr;
  if (check_mirror) {
    msum = ctx.take<unsigned long long>(1);
    zero_words(ctx, msum, sizeof(unsigned long long));
    mirror->dev = msum;
    mirror->queued = true;
  }

  auto global_csc = [&](const int32_t **cp, const int32_t **ri) {
    // Reference: sporder/src/common/csr2csc.h:49-59.
    if (is_symmetric) {
      *cp = d_ptr;
      *ri = d_ind;
      return;
    }
    int32_t *p = ctx.take<int32_t>(static_cast<size_t>(n) + 1);
    int32_t *r = ctx.take<int32_t>(static_cast<size_t>(nnz));
    csr2csc(ctx, n, nnz, d_ptr, d_ind, p, r);
    *cp = p;
    *ri = r;
  };

  if (!local) {
    const int32_t *cp, *ri;
    t_csc->begin(ctx.stream);
    global_csc(&cp, &ri);
    t_csc->end(ctx.stream);
    t_sim->begin(ctx.stream);
    chunk_sketch_top_k(ctx, n, nnz, k, chunk_size, m_cap, d_ptr, d_ind, cp, ri, table,
                       nullptr, nullptr, nullptr, row_valid);
    t_sim->end(ctx.stream);
    return;
  }

  // Chunks are classified and the three list lengths read back; then the
  // sketch paths that have work, which write disjoint table rows, run
  // concurrently: tier 2 (mid-size chunks) on side stream 1, the global-CSC
  // path (large chunks, whose hub rows set the critical path on power-law
  // inputs) on side stream 0 (its largest chunk first, the other chunks' run
  // search and sketch on side stream 2), tier 1 on the library stream.  Tier
  // 1's workgroups take two per CU and leave no room for tier 2's, whose
  // workgroups need a whole CU's LDS.  When tier 1 has at most one chunk per
  // CU it is launched first, over its list: it then holds at most half of the
  // CUs for the length of one chunk, and the tier-2 workgroups placed there
  // late claim fewer chunks (launched after tier 2, it waited for tier 2's
  // last workgroups and ran alone at the end: 2.2 ms of C5's 25.7 ms).  With
  // more tier-1 chunks tier 2 is launched first, and tier 1 waits until the
  // global path's run search is done and its sketch, whose first rows are the
  // heaviest chunk's, is queued.  The transpose of a non-symmetric matrix is
  // built only when the global path has chunks.
  t_sim->begin(ctx.stream);
  chunk_local_classify(ctx, n, chunk_size, d_ptr, lists, counts, is_symmetric);
  int32_t *h_counts = ctx.host_words;
  SP_HIP(hipMemcpyAsync(h_counts, counts, 3 * sizeof(int32_t), hipMemcpyDeviceToHost,
                        ctx.stream));
  ctx.sync();
  const bool run_t2 = h_counts[0] > 0, run_global = h_counts[1] > 0;
  const int64_t t1_len = h_counts[2];
  const bool t1_first = (run_t2 || run_global) && t1_len <= ctx.num_cus;
  if (run_t2) fork_side(ctx, 1);
  if (run_global) fork_side(ctx, 0);
  if (t1_first) {
    chunk_local_sketch_top_k(ctx, n, k, chunk_size, m_cap, d_ptr, d_ind, table, lists, counts,
                             1, row_valid, msum, t1_len);
  }
  if (run_t2) {
    OnStream on(ctx, ctx.side[1]);
    chunk_local_sketch_top_k(ctx, n, k, chunk_size, m_cap, d_ptr, d_ind, table, lists, counts,
                             2, row_valid, msum);
  }
  if (run_global) {
    OnStream on(ctx, ctx.side[0]);
    const int32_t *cp, *ri;
    t_csc->begin(ctx.stream);
    global_csc(&cp, &ri);
    t_csc->end(ctx.stream);
    chunk_sketch_top_k(ctx, n, nnz, k, chunk_size, m_cap, d_ptr, d_ind, cp, ri, table,
                       lists + chunks, counts + 1, t1_first ? nullptr : ctx.prep_ev, row_valid,
                       h_counts[1]);
  } else {
    t_csc->begin(ctx.stream);
    t_csc->end(ctx.stream);
  }
  if (!t1_first) {
    if (run_global) SP_HIP(hipStreamWaitEvent(ctx.stream, ctx.prep_ev, 0));
    chunk_local_sketch_top_k(ctx, n, k, chunk_size, m_cap, d_ptr, d_ind, table, lists, counts,
                             1, row_valid, msum);
  }
  // The global path's rows' mirror check, behind tier 1 on the library
  // stream: ahead of the global path's other chunks (on side stream 2) it held
  // their run search back 3.3 ms on C5.
  if (run_global && msum != nullptr) {
    chunk_mirror_check(ctx, n, chunk_size, d_ptr, d_ind, lists + chunks, counts + 1,
                       h_counts[1], msum);
  }
  if (run_t2) join_side(ctx, 1);
  if (run_global) join_side(ctx, 0);
  t_sim->end(ctx.stream);
}


// Shared body of csg and cg: the top-k table with `sketch_chunk` rows per
// sketch chunk, then the greedy chain over chunks of `chain_chunk` rows.
// Copies the chain counters and table totals to the host when `want_stats`
// and reads the three stage spans when `want_timing`; ends in one
// synchronize.
struct SeriationOut {
  ChainCounters hc{};
  TopKTotals ht{};
  float csr2csc_ms = 0.0f, similarity_ms = 0.0f, chunk_greedy_ms = 0.0f;
};

SeriationOut seriate_pass(Context &ctx, int32_t n, int32_t nnz, const int32_t *d_ptr,
                          const int32_t *d_ind, bool is_symmetric, int32_t k, int32_t m_cap,
                          int32_t sketch_chunk, int32_t chain_chunk, int32_t *d_new_order,
                          bool want_stats, bool want_timing, bool allow_local,
                          bool *redo) {
  const int64_t num_chunks = ceil_div64(n, chain_chunk);
  const int32_t rows_max = static_cast<int32_t>(std::min<int64_t>(chain_chunk, n));
  // The compact chain packs a staged entry's slice position into 20 bits, so
  // it takes chunks of at most kGreedyCompactRows rows whose slice holds at
  // most 2^20 table entries (k up to 256 at 4096 rows); larger slices (k up
  // to 512 is valid) take the general kernel.
  const bool compact = rows_max <= kGreedyCompactRows &&
                       static_cast<int64_t>(rows_max) * k <= (int64_t{1} << 20);
  const int32_t words = static_cast<int32_t>(ceil_div64(rows_max, 32));
  // General greedy: bitmap in LDS when small enough, else in the workspace.
  const size_t lds_need = static_cast<size_t>(words) * 4u;
  const bool bitmap_lds = lds_need <= 64u * 1024u && lds_need <= ctx.lds_per_block;
  const int general_wpb =
      bitmap_lds ? static_cast<int>(std::max<size_t>(
                       1, std::min<size_t>(kGreedyWaves, (64u * 1024u) / std::max<size_t>(lds_need, 1))))
                 : kGreedyWaves;

  size_t need = table_ws_bytes(n, nnz, k, sketch_chunk, is_symmetric) +
                ws_bytes<ChainCounters>(1) + ws_bytes<TopKTotals>(1);
  // About 20 KiB of LDS per chunk at chain_chunk 1024, so that several chunks
  // share a CU.  When there are at most two chunks per CU that LDS would sit
  // idle: the wide variant stages up to 8192 entries (about 70 KiB), so that
  // slices with several in-chunk entries per row still walk from LDS.
  constexpr int32_t kNarrowCap = 8 * kGreedyBlock, kWideCap = 32 * kGreedyBlock;
  const bool wide = compact && num_chunks <= 2 * static_cast<int64_t>(ctx.num_cus) &&
                    static_cast<int64_t>(rows_max) * k > kNarrowCap &&
                    greedy_compact_lds(rows_max, kWideCap) <= ctx.lds_per_block;
  // With many chunks the compact chain can stage only the valid prefix of each
  // table row, from the counts the sketch writes (held as bytes in LDS); a
  // launch of a few chunks is latency-bound and does not use them.
  const bool use_row_valid = compact && !wide && k <= 255;
  // Packed walks (no statistics: the walk then needs no weights) hold up to
  // kPackedCap entries in a region of 32 KiB at chain_chunk 1024, k 16, which
  // would cost the other chunks occupancy: the chain is split over two
  // launches by each slice's valid entries, the packed one taking the slices
  // past the 64-bit staging capacity that it can hold.
  const int32_t packed_cap =
      (use_row_valid && !want_stats && k <= kPackedMaxK)
          ? static_cast<int32_t>(std::min<int64_t>(static_cast<int64_t>(rows_max) * k, kPackedCap))
          : 0;
  if (use_row_valid) need += ws_bytes<int32_t>(static_cast<size_t>(n));
  if (!compact && !bitmap_lds) need += ws_bytes<uint32_t>(static_cast<size_t>(num_chunks) * words);
  ctx.reserve(need);
  uint64_t *table = ctx.take<uint64_t>(static_cast<size_t>(n) * k);
  ChainCounters *counters = ctx.take<ChainCounters>(1);
  TopKTotals *totals = ctx.take<TopKTotals>(1);
  uint32_t *gbitmap = (!compact && !bitmap_lds)
                          ? ctx.take<uint32_t>(static_cast<size_t>(num_chunks) * words)
                          : nullptr;
  int32_t *row_valid = use_row_valid ? ctx.take<int32_t>(static_cast<size_t>(n)) : nullptr;

  EventSpan t_csc, t_sim, t_greedy;
  t_csc.create(want_timing);
  t_sim.create(want_timing);
  t_greedy.create(want_timing);

  if (want_stats) {
    zero_words(ctx, counters, sizeof(ChainCounters));
    zero_words(ctx, totals, sizeof(TopKTotals));
  }

  MirrorCheck mirror;
  build_table(ctx, n, nnz, d_ptr, d_ind, is_symmetric, k, m_cap, sketch_chunk, table, &t_csc,
              &t_sim, &mirror, allow_local, row_valid);
  if (want_stats) top_k_stats(ctx, n, k, table, totals);

  t_greedy.begin(ctx.stream);
  if (compact) {
    const int32_t entry_cap = wide ? kWideCap : kNarrowCap;
    const dim3 grid(static_cast<unsigned>(num_chunks));
    ChainCounters *cnt = want_stats ? counters : nullptr;
    if (wide) {
      greedy_compact_kernel<32><<<grid, kGreedyBlock, greedy_compact_lds(rows_max, entry_cap),
                                  ctx.stream>>>(n, k, chain_chunk, table, d_new_order, cnt,
                                                rows_max, entry_cap, 0, 0, 0, 0, row_valid);
      SP_LAUNCH_CHECK();
    } else {
      // The narrow launch packs slices up to what its own entry region holds
      // as 16-bit entries (4 * entry_cap); the packed launch, with the larger
      // region, follows it and takes the slices between that and packed_cap.
      // Each launch skips the other's chunks after summing their valid
      // counts.  (Run beside each other on two streams, the pair was faster
      // on inputs whose chunks fall on both sides but slower on those whose
      // chunks are all packed, and the fork cost every call about 15 us.)
      const int32_t narrow_packed = std::min(packed_cap, 4 * entry_cap);
      const bool split = packed_cap > narrow_packed;
      const int32_t band_lo = std::max(entry_cap, narrow_packed);
      const int32_t band_hi = split ? packed_cap : 0;
      greedy_compact_kernel<8><<<grid, kGreedyBlock,
                                 greedy_compact_lds(rows_max, entry_cap, narrow_packed),
                                 ctx.stream>>>(n, k, chain_chunk, table, d_new_order, cnt,
                                               rows_max, entry_cap, narrow_packed, band_lo,
                                               band_hi, 0, row_valid);
      SP_LAUNCH_CHECK();
      if (split) {
        greedy_compact_kernel<8>
            <<<grid, kGreedyBlock, greedy_compact_lds(rows_max, entry_cap, packed_cap),
               ctx.stream>>>(n, k, chain_chunk, table, d_new_order, cnt, rows_max, entry_cap,
                             packed_cap, band_lo, band_hi, 1, row_valid);
        SP_LAUNCH_CHECK();
      }
    }
  } else {
    int64_t blocks = ceil_div64(num_chunks, general_wpb);
    size_t lds = bitmap_lds ? static_cast<size_t>(general_wpb) * words * 4u : 0;
    greedy_kernel<<<dim3(static_cast<unsigned>(blocks)), general_wpb * kWave, lds,
                    ctx.stream>>>(n, k, chain_chunk, static_cast<int32_t>(num_chunks), table,
                                  d_new_order, want_stats ? counters : nullptr, gbitmap, words,
                                  bitmap_lds ? 1 : 0);
    SP_LAUNCH_CHECK();
  }
  t_greedy.end(ctx.stream);

  SeriationOut out;
  if (want_stats) {
    SP_HIP(hipMemcpyAsync(&out.hc, counters, sizeof(out.hc), hipMemcpyDeviceToHost,
                          ctx.stream));
    SP_HIP(hipMemcpyAsync(&out.ht, totals, sizeof(out.ht), hipMemcpyDeviceToHost,
                          ctx.stream));
  }
  mirror_collect(ctx, mirror);
  ctx.sync();
  *redo = mirror_failed(ctx, mirror);
  if (want_timing) {
    out.csr2csc_ms = t_csc.ms();
    out.similarity_ms = t_sim.ms();
    out.chunk_greedy_ms = t_greedy.ms();
  }
  t_csc.destroy();
  t_sim.destroy();
  t_greedy.destroy();
  return out;
}

// One seriation; a call with is_symmetric whose pattern fails the mirror
// check is run again with every sketch chunk on the global path, which
// rewrites the order, counters and spans.
SeriationOut seriate(Context &ctx, int32_t n, int32_t nnz, const int32_t *d_ptr,
                     const int32_t *d_ind, bool is_symmetric, int32_t k, int32_t m_cap,
                     int32_t sketch_chunk, int32_t chain_chunk, int32_t *d_new_order,
                     bool want_stats, bool want_timing) {
  bool redo = false;
  SeriationOut out = seriate_pass(ctx, n, nnz, d_ptr, d_ind, is_symmetric, k, m_cap,
                                  sketch_chunk, chain_chunk, d_new_order, want_stats,
                                  want_timing, true, &redo);
  if (redo) {
    out = seriate_pass(ctx, n, nnz, d_ptr, d_ind, is_symmetric, k, m_cap, sketch_chunk,
                       chain_chunk, d_new_order, want_stats, want_timing, false, &redo);
  }
  return out;
}

} // namespace

void top_k_stats(Context &ctx, int32_t n, int32_t k, const uint64_t *d_table,
                 TopKTotals *d_totals) {
  int g = ctx.grid_for(ceil_div64(n, 256), 256, 4);
  top_k_stats_kernel<<<g, 256, 0, ctx.stream>>>(n, k, d_table, d_totals);
  SP_LAUNCH_CHECK();
}

} // namespace sporder_hip

using namespace sporder_hip;

extern "C" {

void sporder_chunk_similarity_greedy(sporder_context_t h, int32_t n,
                                     int32_t nnz, const int32_t *d_ptr,
                                     const int32_t *d_ind, bool is_symmetric,
                                     int32_t k, float oversampling,
                                     int32_t chunk_size, int32_t *d_new_order,
                                     sporder_csg_timing_t *timing,
                                     sporder_csg_stats_t *stats) {
  auto wall0 = std::chrono::steady_clock::now();
  SP_EXPECT(h != nullptr, "null context");
  SP_EXPECT(n >= 1 && nnz >= 0, "expect n >= 1 and nnz >= 0");
  Context &ctx = h->impl;
  // Defaults: reference sporder/src/sporder.cpp:147-161.
  if (k <= 0) k = std::min(256, std::max(16, 1 * (nnz / n)));
  if (oversampling <= 0.0f) oversampling = 4.0f;
  if (chunk_size <= 0) chunk_size = 1024;
  validate_sketch_args(k, oversampling, chunk_size);
  const int32_t m_cap = sketch_m(k, oversampling);
  if (stats) {
    stats->k_used = k;
    stats->m_used = m_cap;
    stats->chunk_size_used = chunk_size;
  }
  const SeriationOut r = seriate(ctx, n, nnz, d_ptr, d_ind, is_symmetric, k, m_cap, chunk_size,
                                 chunk_size, d_new_order, stats != nullptr, timing != nullptr);
  if (stats) {
    // Reference: sporder/src/csg/stats_collector.cu:43-63.
    stats->avg_degree = static_cast<double>(r.ht.total_degree) / n;
    stats->avg_edge_weight =
        r.ht.total_degree > 0 ? r.ht.total_weight / static_cast<double>(r.ht.total_degree)
                              : 0.0;
    stats->zero_degree_rows = r.ht.zero_degree_rows;
    stats->chain_restarts = r.hc.restarts;
    stats->avg_followed_weight = r.hc.links > 0 ? r.hc.link_weight_sum / r.hc.links : 0.0;
  }
  if (timing) {
    timing->csr2csc_ms = r.csr2csc_ms;
    timing->similarity_ms = r.similarity_ms;
    timing->chunk_greedy_ms = r.chunk_greedy_ms;
    timing->wall_ms = std::chrono::duration<double, std::milli>(
                          std::chrono::steady_clock::now() - wall0)
                          .count();
  }
}

void sporder_chunk_greedy(sporder_context_t h, int32_t n, int32_t nnz, const int32_t *d_ptr,
                          const int32_t *d_ind, bool is_symmetric, int32_t k,
                          float oversampling, int32_t chunk_size, int32_t *d_new_order,
                          sporder_cg_timing_t *timing, sporder_cg_stats_t *stats) {
  auto wall0 = std::chrono::steady_clock::now();
  SP_EXPECT(h != nullptr, "null context");
  SP_EXPECT(n >= 1 && nnz >= 0, "expect n >= 1 and nnz >= 0");
  Context &ctx = h->impl;
  // Defaults: reference sporder/src/sporder.cpp:113-125.
  if (k <= 0) k = std::min(256, std::max(16, 1 * (nnz / n)));
  if (oversampling <= 0.0f) oversampling = 4.0f;
  if (chunk_size <= 0) chunk_size = 1024;
  // The global sketch is the chunked one with a single chunk of n rows
  // (reference sporder/src/common/similarity_top_k.cu:10-51 scans every row
  // of each column; the chunk filter [0, n) keeps them all).
  validate_sketch_args(k, oversampling, n);
  const int32_t m_cap = sketch_m(k, oversampling);
  if (stats) {
    stats->k_used = k;
    stats->m_used = m_cap;
    stats->chunk_size_used = chunk_size;
  }
  const SeriationOut r = seriate(ctx, n, nnz, d_ptr, d_ind, is_symmetric, k, m_cap, n,
                                 chunk_size, d_new_order, stats != nullptr, timing != nullptr);
  if (stats) {
    // Reference: sporder/src/cg/stats_collector.cu:45-72.
    stats->avg_degree = static_cast<double>(r.ht.total_degree) / n;
    stats->avg_edge_weight =
        r.ht.total_degree > 0 ? r.ht.total_weight / static_cast<double>(r.ht.total_degree)
                              : 0.0;
    stats->zero_degree_rows = r.ht.zero_degree_rows;
    stats->chain_restarts = r.hc.restarts;
    stats->avg_followed_weight = r.hc.links > 0 ? r.hc.link_weight_sum / r.hc.links : 0.0;
    const double cut =
        r.ht.total_weight > 0.0 ? 1.0 - r.hc.in_chunk_weight / r.ht.total_weight : 0.0;
    stats->cut_weight_fraction = std::min(1.0, std::max(0.0, cut));
  }
  if (timing) {
    timing->csr2csc_ms = r.csr2csc_ms;
    timing->similarity_ms = r.similarity_ms;
    timing->chunk_greedy_ms = r.chunk_greedy_ms;
    timing->wall_ms = std::chrono::duration<double, std::milli>(
                          std::chrono::steady_clock::now() - wall0)
                          .count();
  }
}

void sporder_chunk_similarity_top_k(sporder_context_t h, int32_t n, int32_t nnz,
                                    const int32_t *d_ptr, const int32_t *d_ind,
                                    bool is_symmetric, int32_t k,
                                    float oversampling, int32_t chunk_size,
                                    int32_t *d_indices, float *d_weights) {
  SP_EXPECT(h != nullptr, "null context");
  SP_EXPECT(n >= 1 && nnz >= 0, "expect n >= 1 and nnz >= 0");
  validate_sketch_args(k, oversampling, chunk_size);
  Context &ctx = h->impl;
  // A second pass, on the global path, when is_symmetric fails the mirror check.
  for (bool allow_local = true;; allow_local = false) {
    ctx.reserve(table_ws_bytes(n, nnz, k, chunk_size, is_symmetric));
    uint64_t *table = ctx.take<uint64_t>(static_cast<size_t>(n) * k);
    EventSpan off_a, off_b;
    MirrorCheck mirror;
    build_table(ctx, n, nnz, d_ptr, d_ind, is_symmetric, k, sketch_m(k, oversampling),
                chunk_size, table, &off_a, &off_b, &mirror, allow_local);
    int64_t count = static_cast<int64_t>(n) * k;
    int g = ctx.grid_for(ceil_div64(count, 256), 256, 4);
    unpack_table_kernel<<<g, 256, 0, ctx.stream>>>(count, table, d_indices, d_weights);
    SP_LAUNCH_CHECK();
    mirror_collect(ctx, mirror);
    ctx.sync();
    if (!mirror_failed(ctx, mirror)) break;
  }
}

void sporder_similarity_graph(sporder_context_t h, int32_t n, int32_t nnz,
                              const int32_t *d_ptr, const int32_t *d_ind,
                              bool is_symmetric, int32_t k, float oversampling,
                              int32_t *d_indices, float *d_weights,
                              sporder_sim_timing_t *timing,
                              sporder_sim_stats_t *stats) {
  auto wall0 = std::chrono::steady_clock::now();
  SP_EXPECT(h != nullptr, "null context");
  SP_EXPECT(n >= 1 && nnz >= 0, "expect n >= 1 and nnz >= 0");
  Context &ctx = h->impl;
  // Defaults: reference sporder/src/sporder.cpp:75-85.
  if (k <= 0) k = std::min(32, std::max(16, 2 * (nnz / n)));
  if (oversampling <= 0.0f) oversampling = 2.0f;
  // One chunk spanning every row is the global sketch of
  // sporder/src/common/similarity_top_k.cu:10-51.
  validate_sketch_args(k, oversampling, n);
  const int32_t m_cap = sketch_m(k, oversampling);
  if (stats) {
    stats->k_used = k;
    stats->m_used = m_cap;
  }
  EventSpan t_csc, t_sim, t_unpack;
  t_csc.create(timing != nullptr);
  t_sim.create(timing != nullptr);
  t_unpack.create(timing != nullptr);
  TopKTotals ht{};
  // A second pass, on the global path, when is_symmetric fails the mirror check.
  for (bool allow_local = true;; allow_local = false) {
    ctx.reserve(table_ws_bytes(n, nnz, k, n, is_symmetric) + ws_bytes<TopKTotals>(1));
    uint64_t *table = ctx.take<uint64_t>(static_cast<size_t>(n) * k);
    TopKTotals *totals = ctx.take<TopKTotals>(1);
    MirrorCheck mirror;
    build_table(ctx, n, nnz, d_ptr, d_ind, is_symmetric, k, m_cap, n, table, &t_csc, &t_sim,
                &mirror, allow_local);
    if (stats) {
      zero_words(ctx, totals, sizeof(TopKTotals));
      top_k_stats(ctx, n, k, table, totals);
    }
    int64_t count = static_cast<int64_t>(n) * k;
    int g = ctx.grid_for(ceil_div64(count, 256), 256, 4);
    t_unpack.begin(ctx.stream);
    unpack_table_kernel<<<g, 256, 0, ctx.stream>>>(count, table, d_indices, d_weights);
    SP_LAUNCH_CHECK();
    t_unpack.end(ctx.stream);
    if (stats) {
      SP_HIP(hipMemcpyAsync(&ht, totals, sizeof(ht), hipMemcpyDeviceToHost, ctx.stream));
    }
    mirror_collect(ctx, mirror);
    ctx.sync();
    if (!mirror_failed(ctx, mirror)) break;
  }
  if (timing) {
    timing->csr2csc_ms = t_csc.ms();
    timing->similarity_ms = t_sim.ms();
    timing->unpack_ms = t_unpack.ms();
    timing->wall_ms = std::chrono::duration<double, std::milli>(
                          std::chrono::steady_clock::now() - wall0)
                          .count();
  }
  if (stats) {
    stats->avg_degree = static_cast<double>(ht.total_degree) / n;
    stats->avg_edge_weight =
        ht.total_degree > 0 ? ht.total_weight / static_cast<double>(ht.total_degree)
                            : 0.0;
    stats->zero_degree_rows = ht.zero_degree_rows;
  }
  t_csc.destroy();
  t_sim.destroy();
  t_unpack.destroy();
}

} // extern "C"
