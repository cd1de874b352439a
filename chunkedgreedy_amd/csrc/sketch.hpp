// sketch.hpp -- the wave64 space-saving sketch shared by the csg kernels.
//
// Semantics: reference sporder/src/common/warp_spacesaving.cuh:12-151 and the
// arg-reductions of sporder/src/common/cuda_util.cuh:66-87.  The reference
// keeps M = 32*CELLS slots in one 32-lane warp: logical lane L owns cells
// c = 0..CELLS-1.  Here one wave64 holds the slots of one row: physical lane p
// holds logical lane L = p & 31 and the cells c = 2j + (p >> 5),
// j = 0..ceil(CELLS/2)-1.  Every tie rule of the reference depends only on
// (L, c), so the arrangement is free:
//   - a new key goes to the first empty slot in order s = L*CELLS + c (slots
//     never empty again), a wave-uniform counter instead of find(-1) + ballot;
//   - eviction takes the minimum of (weight, c*32 + L): a DPP minimum of the
//     weight bits, then ballots in tie order; the new key inherits the evicted
//     weight;
//   - output merges the per-logical-lane selection-sorted lists, largest head
//     weight first (DPP maximum), ties to the smaller logical lane.  That
//     order is (weight descending, logical lane, list position); for at most
//     four cells per logical lane it is produced by one bitonic sort of
//     (weight, position) keys over one or two registers of the wave.
#pragma once

#include "common.hpp"

namespace sporder_hip {

__device__ __forceinline__ int32_t lower_bound_dev(const int32_t *a, int32_t lo,
                                                   int32_t hi, int32_t t) {
  while (lo < hi) {
    int32_t mid = lo + (hi - lo) / 2;
    if (a[mid] < t) {
      lo = mid + 1;
    } else {
      hi = mid;
    }
  }
  return lo;
}

// lower_bound_dev for an answer expected near `lo`: probe lo, lo+1, lo+3,
// lo+7, ... until an element >= t (or hi) is passed, then search the last
// doubling interval.  log2(distance) probes instead of log2(hi - lo).
__device__ __forceinline__ int32_t gallop_lower_bound(const int32_t *a, int32_t lo,
                                                      int32_t hi, int32_t t) {
  int32_t b = 1;
  while (lo + b < hi && a[lo + b - 1] < t) b <<= 1;
  // a[lo + b/2 - 1] < t when b > 1, and a[lo + b - 1] >= t unless lo + b >= hi.
  return lower_bound_dev(a, lo + (b >> 1), lo + b < hi ? lo + b : hi, t);
}

// Per lane: `a` where the lane's bit of the wave mask is set, else `b`.  One
// v_cndmask with the mask as its lane condition, written out so that the
// compiler keeps it a select: left to itself it may turn a select on a
// sparse mask into an execution-masked region behind a branch.  The mask is
// wave-uniform (built from ballots); readfirstlane states that to the
// compiler, which drops it where it already holds the mask in scalar
// registers.
__device__ __forceinline__ int32_t mask_select(uint64_t mask, int32_t a, int32_t b) {
  const uint64_t m =
      static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int32_t>(mask))) |
      (static_cast<uint64_t>(static_cast<uint32_t>(
           __builtin_amdgcn_readfirstlane(static_cast<int32_t>(mask >> 32))))
       << 32);
  int32_t r;
  asm("v_cndmask_b32_e64 %0, %2, %1, %3" : "=v"(r) : "v"(a), "v"(b), "s"(m));
  return r;
}

// Bitonic sort of 64-bit keys held as (hi, lo) pairs, one per lane and
// register: element x = 64*q + lane sits in register q.  Step (kk, j) pairs x
// with x ^ j; the smaller key goes to the lower x of a pair in an ascending
// block ((x & kk) == 0) and to the upper x in a descending one.
//
// Lanes of register q (base = 64*q) that keep the smaller key in step (kk, j)
// for j < 64, where the partner is lane ^ j of the same register.
constexpr uint64_t bitonic_keep_min(int kk, int j, int base) {
  uint64_t m = 0;
  for (int l = 0; l < 64; ++l) {
    if (((l & j) != 0) == (((base + l) & kk) != 0)) m |= 1ull << l;
  }
  return m;
}

// Step (KK, J < 64) on the register of base BASE.  A lane takes its
// partner's key when the partner is larger and the lane keeps the maximum,
// or is not larger and the lane keeps the minimum (taking an equal key
// changes nothing): one compare and the step's constant mask.
template <int KK, int J, int BASE>
__device__ __forceinline__ void bitonic_step64(uint32_t &hi, uint32_t &lo) {
  const uint32_t ph = lane_xor_u32(hi, J), pl = lane_xor_u32(lo, J);
  const uint64_t mine = (static_cast<uint64_t>(hi) << 32) | lo;
  const uint64_t other = (static_cast<uint64_t>(ph) << 32) | pl;
  constexpr uint64_t kKeepMin = bitonic_keep_min(KK, J, BASE);
  const uint64_t take = ballot(other > mine) ^ kKeepMin;
  hi = static_cast<uint32_t>(mask_select(take, static_cast<int32_t>(ph), static_cast<int32_t>(hi)));
  lo = static_cast<uint32_t>(mask_select(take, static_cast<int32_t>(pl), static_cast<int32_t>(lo)));
}

// Steps J = J0, J0/2, ..., 1 (all below 64) of stage KK on one register.
template <int KK, int J0, int BASE>
__device__ __forceinline__ void bitonic_steps64(uint32_t &hi, uint32_t &lo) {
  bitonic_step64<KK, J0, BASE>(hi, lo);
  if constexpr (J0 > 1) bitonic_steps64<KK, J0 / 2, BASE>(hi, lo);
}

// Ascending sort of the first `span` elements of one register, whose lanes
// at or past `span` hold the largest key: the stages run up to the first
// block size that covers span (blocks of every stage up to kk are sorted,
// the first one ascending), so lanes [0, span) end in order.  span is
// wave-uniform; MAXKK (32 or 64) is the largest stage the caller needs.
template <int MAXKK>
__device__ __forceinline__ void bitonic_sort_prefix64(uint32_t &hi, uint32_t &lo, int span) {
  if (span > 1) {
    bitonic_steps64<2, 1, 0>(hi, lo);
    if (span > 2) {
      bitonic_steps64<4, 2, 0>(hi, lo);
      if (span > 4) {
        bitonic_steps64<8, 4, 0>(hi, lo);
        if (span > 8) {
          bitonic_steps64<16, 8, 0>(hi, lo);
          if (span > 16) {
            bitonic_steps64<32, 16, 0>(hi, lo);
            if constexpr (MAXKK > 32) {
              if (span > 32) bitonic_steps64<64, 32, 0>(hi, lo);
            }
          }
        }
      }
    }
  }
}

// Ascending sort of all 128 elements of two registers.
__device__ __forceinline__ void bitonic_sort128(uint32_t (&hi)[2], uint32_t (&lo)[2]) {
  bitonic_steps64<2, 1, 0>(hi[0], lo[0]);
  bitonic_steps64<2, 1, 64>(hi[1], lo[1]);
  bitonic_steps64<4, 2, 0>(hi[0], lo[0]);
  bitonic_steps64<4, 2, 64>(hi[1], lo[1]);
  bitonic_steps64<8, 4, 0>(hi[0], lo[0]);
  bitonic_steps64<8, 4, 64>(hi[1], lo[1]);
  bitonic_steps64<16, 8, 0>(hi[0], lo[0]);
  bitonic_steps64<16, 8, 64>(hi[1], lo[1]);
  bitonic_steps64<32, 16, 0>(hi[0], lo[0]);
  bitonic_steps64<32, 16, 64>(hi[1], lo[1]);
  bitonic_steps64<64, 32, 0>(hi[0], lo[0]);  // ascending block
  bitonic_steps64<64, 32, 64>(hi[1], lo[1]); // descending block
  // Stage 128, j = 64: the partners share a lane; register 0 keeps the
  // smaller key.
  {
    const uint64_t a = (static_cast<uint64_t>(hi[0]) << 32) | lo[0];
    const uint64_t b = (static_cast<uint64_t>(hi[1]) << 32) | lo[1];
    const bool swap = a > b;
    const uint32_t h0 = hi[0], l0 = lo[0];
    hi[0] = swap ? hi[1] : hi[0];
    lo[0] = swap ? lo[1] : lo[0];
    hi[1] = swap ? h0 : hi[1];
    lo[1] = swap ? l0 : lo[1];
  }
  bitonic_steps64<128, 32, 0>(hi[0], lo[0]);
  bitonic_steps64<128, 32, 64>(hi[1], lo[1]);
}

// Space-saving sketch of capacity 32*CELLS spread over one wave64.
template <int CELLS> struct WaveSketch {
  static constexpr int LC = (CELLS + 1) / 2; // cells held per physical lane
  static constexpr int M = 32 * CELLS;
  int32_t key[LC];
  float wt[LC];
  int32_t filled; // wave-uniform: slots taken so far (fill order L*CELLS+c)

  // Physical lane p holds cell c = 2j + (p >> 5); for odd CELLS the upper
  // half of the last j is not a cell.
  static __device__ __forceinline__ bool cell_valid(int j, int lane) {
    return (CELLS % 2 == 0) || j < LC - 1 || lane < 32;
  }

  __device__ __forceinline__ void clear() {
#pragma unroll
    for (int j = 0; j < LC; ++j) {
      key[j] = -1;
      wt[j] = 0.0f;
    }
    filled = 0;
  }

  // Apply one item; k and w are wave-uniform.
  //
  // Every slot write below is a select whose per-lane condition is a wave
  // mask (inverse ballot): the hit masks from the key compares, and for a
  // miss the one-hot mask of the slot's lane, so the slot written costs two
  // selects per cell and no lane compare.  A hit's weight is added only after
  // the hit test, behind a branch: fewer vector instructions per miss, for
  // kernels where many waves share a SIMD and issue slots, not one chain, set
  // the time (the chunk tiers).
  __device__ __forceinline__ void add(int32_t k, float w) {
    if (hit_update<false>(k, w)) return;
    // A miss writes (k, wn) into one slot: the lane of the one-hot mask
    // sel[j] in local cell j.
    uint64_t sel[LC];
    float wn;
    if (filled < M) {
      // Slot s = L*CELLS + c: logical lane L, cell c -> physical lane
      // L + 32*(c & 1), local cell c >> 1.
      const uint32_t f = static_cast<uint32_t>(filled);
      const uint32_t L = f / CELLS, c = f - L * CELLS;
      const uint64_t bit = 1ull << (L + 32u * (c & 1u));
#pragma unroll
      for (int j = 0; j < LC; ++j) sel[j] = (static_cast<uint32_t>(j) == (c >> 1)) ? bit : 0;
      wn = w;
      filled += 1;
    } else {
      // Evict the argmin of (weight, c*32 + L).  With c = 2j + (p >> 5) and
      // L = p & 31, c*32 + L = 64j + p, so ties go to the smallest cell index
      // j and then the lowest physical lane p.  Weights are positive floats
      // (sums of 2/(a+b)), so their bit patterns order like the values.
      const int lane = lane_id();
      uint32_t lmin = 0xFFFFFFFFu;
#pragma unroll
      for (int j = 0; j < LC; ++j) {
        if (cell_valid(j, lane)) lmin = min(lmin, __float_as_uint(wt[j]));
      }
      const uint32_t wmin = wave_min_u32(lmin);
      // The evicted slot holds exactly wmin, so the weight it inherits,
      // wmin + w, is the same value in every lane.
      wn = __uint_as_float(wmin) + w;
      bool found = false;
#pragma unroll
      for (int j = 0; j < LC; ++j) {
        const uint64_t m = ballot(cell_valid(j, lane) && __float_as_uint(wt[j]) == wmin);
        sel[j] = found ? 0 : (m & (~m + 1)); // lowest set lane
        found = found || m != 0;
      }
    }
#pragma unroll
    for (int j = 0; j < LC; ++j) {
      key[j] = mask_select(sel[j], k, key[j]);
      wt[j] = __int_as_float(mask_select(sel[j], __float_as_int(wn), __float_as_int(wt[j])));
    }
  }

  // Apply the items of the lanes set in `mask`, in lane order: item i is
  // (readlane(other, i), readlane(alpha, i)).  The same updates as add() item
  // by item, in two loops: while slots are free a miss fills the next one,
  // afterwards every miss evicts, so neither loop tests the capacity per
  // item; and an eviction looks for the tied minimum only in the first cell
  // that holds the minimum (ties go to the smallest cell index, then lane).
  // A hit's weight is added before the miss test: one taken branch per hit,
  // for a wave whose single long stream is the critical path (one row's items
  // are a dependent chain, and every taken branch lengthens it: the global
  // path's hub rows).
  __device__ __forceinline__ void feed(uint64_t mask, int32_t other, float alpha) {
    if constexpr (CELLS == 4) {
      feed4(mask, other, alpha);
    } else {
      feed_generic(mask, other, alpha);
    }
  }

  // feed() in compiled code, for every capacity.
  __device__ __forceinline__ void feed_generic(uint64_t mask, int32_t other, float alpha) {
    const int lane = lane_id();
    while (mask != 0 && filled < M) {
      const int i = __builtin_ctzll(mask);
      mask &= mask - 1;
      const int32_t k = readlane(other, i);
      const float w = readlane_f(alpha, i);
      if (hit_update<true>(k, w)) continue;
      const uint32_t f = static_cast<uint32_t>(filled);
      const uint32_t L = f / CELLS, c = f - L * CELLS;
      const uint64_t bit = 1ull << (L + 32u * (c & 1u));
#pragma unroll
      for (int j = 0; j < LC; ++j) {
        const uint64_t sel = (static_cast<uint32_t>(j) == (c >> 1)) ? bit : 0;
        key[j] = mask_select(sel, k, key[j]);
        wt[j] = __int_as_float(mask_select(sel, __float_as_int(w), __float_as_int(wt[j])));
      }
      filled += 1;
    }
    while (mask != 0) {
      const int i = __builtin_ctzll(mask);
      mask &= mask - 1;
      const int32_t k = readlane(other, i);
      const float w = readlane_f(alpha, i);
      if (hit_update<true>(k, w)) continue;
      uint32_t lmin = 0xFFFFFFFFu;
#pragma unroll
      for (int j = 0; j < LC; ++j) {
        if (cell_valid(j, lane)) lmin = min(lmin, __float_as_uint(wt[j]));
      }
      const uint32_t wmin = wave_min_u32(lmin);
      const float wn = __uint_as_float(wmin) + w; // the evicted slot holds wmin
      bool found = false;
#pragma unroll
      for (int j = 0; j < LC; ++j) {
        if (!found) {
          const uint64_t m = ballot(cell_valid(j, lane) && __float_as_uint(wt[j]) == wmin);
          if (m != 0) {
            const uint64_t sel = 1ull << __builtin_ctzll(m);
            key[j] = mask_select(sel, k, key[j]);
            wt[j] = __int_as_float(mask_select(sel, __float_as_int(wn), __float_as_int(wt[j])));
            found = true;
          }
        }
      }
    }
  }

  // The chunk tiers' item loop: add() item by item in lane order (the form
  // that measured fastest there for capacities other than 128), or feed4.
  __device__ __forceinline__ void consume(uint64_t mask, int32_t other, float alpha) {
    if constexpr (CELLS == 4) {
      feed4(mask, other, alpha);
    } else {
      while (mask) {
        const int i = __builtin_ctzll(mask);
        add(readlane(other, i), readlane_f(alpha, i));
        mask = clear_bit(mask, i);
      }
    }
  }

  // feed() for CELLS == 4 (M = 128, two cells in every lane: the capacity of
  // csg's default k of 17..32), written as one block of GCN assembly.  The
  // same updates as add() item by item; written out because the compiler's
  // version of the same steps issues more instructions per miss (register
  // copies where the hit and miss paths join, both cells written where one
  // changes, a three-instruction lowest-bit isolation per cell), and the
  // chunk tiers are issue-bound: on a C5-like stream (half the items from
  // 100 hot keys, half from 1000 cold ones) the whole GPU moves 23.0 G
  // items/s through the compiled loop and 27.9 G items/s through this one
  // at four waves per SIMD, with the same slots afterwards.
  //
  // Per item (lane i of the mask, lowest first): k, w by v_readlane; the hit
  // masks h0, h1 of the two cells.  A hit adds w in both cells, each select
  // on its hit mask (one of them is empty): no branch on the cell, which
  // costs a single wave more than the two vector instructions it saves.
  // Each path ends with its own test for a next item and jump back, so a hit
  // takes one taken branch.  A miss while slots are free fills
  // slot s = filled: logical lane s >> 2, cell s & 3, i.e. physical lane
  // (s >> 2) + 32 (s & 1), local cell (s >> 1) & 1, written by v_writelane.
  // A miss on a full sketch takes the DPP minimum of the weight bits (as
  // wave_min_u32), then the first tied lane of cell 0, else of cell 1 (tie
  // order c*32 + L = 64j + p), and writes k there with v_writelane and
  // wmin + w as the lane's own weight plus w (the lane holds exactly wmin).
  //
  // Wait states: the s_nop counts are those the compiler puts between the
  // same instructions (a VALU write of an SGPR before a VALU read of it: 2; a
  // VALU write of a VGPR before a DPP read of it: 2; a DPP write before
  // v_readlane of it: 1).  Lane selects of v_readlane and v_writelane are
  // written by scalar instructions (s_ff1, s_add); the one of v_writelane is
  // M0 (with an SGPR data operand, another SGPR as lane select breaks the
  // one-scalar-operand limit of a VALU instruction), with one wait state
  // after its write; the block saves M0 and restores it at the end.
  // Every lane of the wave must be active.
  __device__ __forceinline__ void feed4(uint64_t mask, int32_t other, float alpha) {
    static_assert(CELLS == 4, "two cells per lane");
    uint32_t i, p, q, kk, ww, wmin;
    uint64_t h0, h1, any, mm, sel;
    float t;
    // Both are wave-uniform; readfirstlane states it, so that the compiler
    // hands them over in scalar registers.
    mask = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int32_t>(mask))) |
           (static_cast<uint64_t>(static_cast<uint32_t>(
                __builtin_amdgcn_readfirstlane(static_cast<int32_t>(mask >> 32))))
            << 32);
    filled = __builtin_amdgcn_readfirstlane(filled);
    uint32_t m0_saved;
    asm volatile(
        "s_mov_b32 %[m0s], m0\n\t"
        "s_cmp_eq_u64 %[mask], 0\n\t"
        "s_cbranch_scc1 9f\n"
        // ---- while slots are free (mask != 0 here)
        "0:\n\t"
        "s_cmp_ge_u32 %[f], 0x80\n\t"
        "s_cbranch_scc1 5f\n\t"
        "s_ff1_i32_b64 %[i], %[mask]\n\t"
        "s_bitset0_b64 %[mask], %[i]\n\t"
        "v_readlane_b32 %[kk], %[other], %[i]\n\t"
        "v_readlane_b32 %[ww], %[alpha], %[i]\n\t"
        "s_nop 0\n\t"
        "v_cmp_eq_u32_e64 %[h0], %[kk], %[k0]\n\t"
        "v_cmp_eq_u32_e64 %[h1], %[kk], %[k1]\n\t"
        "s_or_b64 %[any], %[h0], %[h1]\n\t"
        "s_cbranch_scc0 2f\n\t"
        // hit: the add in both cells, selected by the hit masks (one is empty)
        "v_add_f32_e64 %[t], %[ww], %[w0]\n\t"
        "v_cndmask_b32_e64 %[w0], %[w0], %[t], %[h0]\n\t"
        "v_add_f32_e64 %[t], %[ww], %[w1]\n\t"
        "v_cndmask_b32_e64 %[w1], %[w1], %[t], %[h1]\n\t"
        "s_cmp_lg_u64 %[mask], 0\n\t"
        "s_cbranch_scc1 0b\n\t"
        "s_branch 9f\n"
        // fill slot f: physical lane (f >> 2) + 32 (f & 1), cell (f >> 1) & 1
        "2:\n\t"
        "s_lshr_b32 %[p], %[f], 2\n\t"
        "s_and_b32 %[q], %[f], 1\n\t"
        "s_lshl_b32 %[q], %[q], 5\n\t"
        "s_add_u32 m0, %[p], %[q]\n\t"
        "s_bitcmp1_b32 %[f], 1\n\t"
        "s_cbranch_scc1 3f\n\t"
        "v_writelane_b32 %[k0], %[kk], m0\n\t"
        "v_writelane_b32 %[w0], %[ww], m0\n\t"
        "s_add_u32 %[f], %[f], 1\n\t"
        "s_cmp_lg_u64 %[mask], 0\n\t"
        "s_cbranch_scc1 0b\n\t"
        "s_branch 9f\n"
        "3:\n\t"
        "v_writelane_b32 %[k1], %[kk], m0\n\t"
        "v_writelane_b32 %[w1], %[ww], m0\n\t"
        "s_add_u32 %[f], %[f], 1\n\t"
        "s_cmp_lg_u64 %[mask], 0\n\t"
        "s_cbranch_scc1 0b\n\t"
        "s_branch 9f\n"
        // ---- full: every miss evicts (mask != 0 here)
        "5:\n\t"
        "s_ff1_i32_b64 %[i], %[mask]\n\t"
        "s_bitset0_b64 %[mask], %[i]\n\t"
        "v_readlane_b32 %[kk], %[other], %[i]\n\t"
        "v_readlane_b32 %[ww], %[alpha], %[i]\n\t"
        "s_nop 0\n\t"
        "v_cmp_eq_u32_e64 %[h0], %[kk], %[k0]\n\t"
        "v_cmp_eq_u32_e64 %[h1], %[kk], %[k1]\n\t"
        "s_or_b64 %[any], %[h0], %[h1]\n\t"
        "s_cbranch_scc0 6f\n\t"
        "v_add_f32_e64 %[t], %[ww], %[w0]\n\t"
        "v_cndmask_b32_e64 %[w0], %[w0], %[t], %[h0]\n\t"
        "v_add_f32_e64 %[t], %[ww], %[w1]\n\t"
        "v_cndmask_b32_e64 %[w1], %[w1], %[t], %[h1]\n\t"
        "s_cmp_lg_u64 %[mask], 0\n\t"
        "s_cbranch_scc1 5b\n\t"
        "s_branch 9f\n"
        "6:\n\t"
        "v_min_u32_e32 %[t], %[w0], %[w1]\n\t"
        "s_nop 1\n\t"
        "v_min_u32_dpp %[t], %[t], %[t] quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_min_u32_dpp %[t], %[t], %[t] quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_min_u32_dpp %[t], %[t], %[t] row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_min_u32_dpp %[t], %[t], %[t] row_mirror row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_min_u32_dpp %[t], %[t], %[t] row_bcast:15 row_mask:0xa bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_min_u32_dpp %[t], %[t], %[t] row_bcast:31 row_mask:0xc bank_mask:0xf\n\t"
        "s_nop 0\n\t"
        "v_readlane_b32 %[wmin], %[t], 63\n\t"
        "s_nop 1\n\t"
        "v_cmp_eq_u32_e64 %[mm], %[wmin], %[w0]\n\t"
        "s_cmp_eq_u64 %[mm], 0\n\t"
        "s_cbranch_scc1 7f\n\t"
        "s_ff1_i32_b64 m0, %[mm]\n\t"
        "s_nop 0\n\t"
        "v_writelane_b32 %[k0], %[kk], m0\n\t"
        "s_lshl_b64 %[sel], 1, m0\n\t"
        "v_add_f32_e64 %[t], %[ww], %[w0]\n\t"
        "v_cndmask_b32_e64 %[w0], %[w0], %[t], %[sel]\n\t"
        "s_cmp_lg_u64 %[mask], 0\n\t"
        "s_cbranch_scc1 5b\n\t"
        "s_branch 9f\n"
        "7:\n\t"
        "v_cmp_eq_u32_e64 %[mm], %[wmin], %[w1]\n\t"
        "s_ff1_i32_b64 m0, %[mm]\n\t"
        "s_nop 0\n\t"
        "v_writelane_b32 %[k1], %[kk], m0\n\t"
        "s_lshl_b64 %[sel], 1, m0\n\t"
        "v_add_f32_e64 %[t], %[ww], %[w1]\n\t"
        "v_cndmask_b32_e64 %[w1], %[w1], %[t], %[sel]\n\t"
        "s_cmp_lg_u64 %[mask], 0\n\t"
        "s_cbranch_scc1 5b\n"
        "9:\n\t"
        "s_mov_b32 m0, %[m0s]"
        : [k0] "+v"(key[0]), [k1] "+v"(key[1]), [w0] "+v"(wt[0]), [w1] "+v"(wt[1]),
          [mask] "+s"(mask), [f] "+s"(filled), [t] "=&v"(t), [i] "=&s"(i), [p] "=&s"(p),
          [q] "=&s"(q), [kk] "=&s"(kk), [ww] "=&s"(ww), [wmin] "=&s"(wmin), [h0] "=&s"(h0),
          [h1] "=&s"(h1), [any] "=&s"(any), [mm] "=&s"(mm), [sel] "=&s"(sel),
          [m0s] "=&s"(m0_saved)
        : [other] "v"(other), [alpha] "v"(alpha)
        : "scc");
  }

  // The hit test: true (and the weight added) when k is held.  HIT_FIRST adds
  // the weight with selects before the result is known (feed), otherwise
  // behind the branch on it (add).
  template <bool HIT_FIRST>
  __device__ __forceinline__ bool hit_update(int32_t k, float w) {
    uint64_t hit[LC];
    uint64_t any = 0;
#pragma unroll
    for (int j = 0; j < LC; ++j) {
      hit[j] = ballot(key[j] == k);
      any |= hit[j];
      if (HIT_FIRST) wt[j] = __builtin_amdgcn_inverse_ballot_w64(hit[j]) ? wt[j] + w : wt[j];
    }
    if (any == 0) return false;
    if (!HIT_FIRST) {
#pragma unroll
      for (int j = 0; j < LC; ++j) {
        if (__builtin_amdgcn_inverse_ballot_w64(hit[j])) wt[j] += w;
      }
    }
    return true;
  }

  // Reference select_top_k: per-logical-lane selection sort (strict '>',
  // stop at -1), then up to k rounds emitting the head of the lane with the
  // largest head weight (ties -> smaller lane; exhausted lanes show 0.0f).
  // Writes all k entries of `out` (unused ones as the zero entry).
  __device__ __forceinline__ void select_top_k(int32_t k, uint64_t *out) {
    if constexpr (CELLS <= 2) {
      select_top_k_sorted(k, out);
      return;
    }
    const int lane = lane_id();
    // Gather logical lane L's cells into physical lane L (< 32).
    int32_t fk[CELLS];
    float fw[CELLS];
#pragma unroll
    for (int j = 0; j < LC; ++j) {
      int32_t hk = __shfl(key[j], (lane & 31) + 32, kWave);
      float hw = __shfl(wt[j], (lane & 31) + 32, kWave);
      fk[2 * j] = key[j];
      fw[2 * j] = wt[j];
      if (2 * j + 1 < CELLS) {
        fk[2 * j + 1] = hk;
        fw[2 * j + 1] = hw;
      }
    }
    // Selection sort, literally as the reference (not stable).
#pragma unroll
    for (int i = 0; i < CELLS - 1; ++i) {
      if (fk[i] == -1) break;
      int best = i;
      float bw = fw[i];
#pragma unroll
      for (int j = i + 1; j < CELLS; ++j) {
        if (fk[j] == -1) break;
        if (fw[j] > bw) {
          best = j;
          bw = fw[j];
        }
      }
      if (best != i) {
        // Swap cells i and best (best is a run-time index: select by loop).
        int32_t tk = fk[i];
        float tw = fw[i];
#pragma unroll
        for (int j = i + 1; j < CELLS; ++j) {
          if (j == best) {
            fk[i] = fk[j];
            fw[i] = fw[j];
            fk[j] = tk;
            fw[j] = tw;
          }
        }
      }
    }
    if constexpr (CELLS >= 3 && CELLS <= 4) {
      emit_sorted_lists(k, out, fk, fw);
      return;
    }
    // k-way merge; lane (i & 63) keeps output entry i in register i >> 6.
    // The row has k <= M = 32 * CELLS <= 64 * LC entries (m = (int)(k * ovs)
    // >= k for ovs >= 1, and M rounds m up), so LC registers per lane hold the
    // whole output row; entries past the last emitted one stay zero.
    uint64_t outv[LC];
#pragma unroll
    for (int r = 0; r < LC; ++r) outv[r] = 0;
    for (int32_t i = 0; i < k; ++i) {
      bool live = lane < 32 && fk[0] != -1;
      if (ballot(live) == 0) break;
      // Largest head weight, ties to the smaller lane.  Live heads are
      // positive, exhausted lanes present 0.0f and the upper half-wave holds
      // no logical lane, so bit patterns compare like the weights.
      const uint32_t v = live ? __float_as_uint(fw[0]) : 0u;
      const uint32_t vmax = wave_max_u32(v);
      const int who = __builtin_ctzll(ballot(live && v == vmax));
      const int winner = who;
      int32_t wk = readlane(fk[0], winner);
      float ww = readlane_f(fw[0], winner);
      int slot = i >> 6; // below LC: i < M
      if (lane == (i & 63)) {
#pragma unroll
        for (int r = 0; r < LC; ++r) {
          if (r == slot) outv[r] = pack_wi(wk, ww);
        }
      }
      if (lane == winner) {
#pragma unroll
        for (int j = 0; j < CELLS - 1; ++j) {
          fk[j] = fk[j + 1];
          fw[j] = fw[j + 1];
        }
        fk[CELLS - 1] = -1;
        fw[CELLS - 1] = 0.0f;
      }
    }
#pragma unroll
    for (int r = 0; r < LC; ++r) {
      const int32_t idx = r * 64 + lane;
      if (idx < k) out[idx] = outv[r];
    }
  }

  // The merge of select_top_k for 3 <= CELLS <= 4, from the selection-sorted
  // lists fk/fw of logical lane L (held by physical lane L < 32).  The merge
  // emits every entry of weight above w before any of weight w (each list
  // descends), and among equal weights drains the smallest logical lane's
  // run first, in list order: output order is (weight descending, L, list
  // position pos).  Entry e = L*CELLS + pos is placed at element x = e of two
  // registers (x = 64*q + lane) with the key (~weight bits, e); live entries
  // are a prefix of e (slots fill logical lane by logical lane, and the sort
  // keeps a lane's live cells first), so rows of at most 64 live entries sort
  // register 0 alone, up to the block that covers them.  Element i of the
  // sorted keys is output entry i.
  __device__ __forceinline__ void emit_sorted_lists(int32_t k, uint64_t *out,
                                                    const int32_t (&fk)[CELLS],
                                                    const float (&fw)[CELLS]) {
    static_assert(CELLS >= 3 && CELLS <= 4, "two registers of 64 elements");
    const int lane = lane_id();
    int32_t sk[2];
    uint32_t hi[2], lo[2];
    uint64_t lm[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      // Element x = 64q + lane holds e = x: list entry pos of logical lane L.
      const int e = 64 * q + lane;
      const int L = e / CELLS, pos = e - L * CELLS;
      const int src = L & 31;
      int32_t kx = -1;
      float wx = 0.0f;
#pragma unroll
      for (int p = 0; p < CELLS; ++p) {
        const int32_t kp = __shfl(fk[p], src, kWave);
        const float wp = __shfl(fw[p], src, kWave);
        if (pos == p) {
          kx = kp;
          wx = wp;
        }
      }
      if (L >= 32) kx = -1; // past M = 32*CELLS (CELLS == 3)
      const bool live = kx != -1;
      sk[q] = kx;
      lm[q] = ballot(live);
      hi[q] = live ? ~__float_as_uint(wx) : 0xFFFFFFFFu;
      lo[q] = live ? static_cast<uint32_t>(e) : 0xFFFFFFFFu;
    }
    const int n_live = __popcll(lm[0]) + __popcll(lm[1]);
    if (lm[1] != 0) {
      bitonic_sort128(hi, lo);
    } else {
      bitonic_sort_prefix64<64>(hi[0], lo[0], lm[0] ? 64 - __builtin_clzll(lm[0]) : 0);
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int i = 64 * q + lane;
      const int e = static_cast<int>(lo[q] & 127u);
      const int32_t k0 = __shfl(sk[0], e & 63, kWave);
      const int32_t k1 = __shfl(sk[1], e & 63, kWave);
      const int32_t idx = e < 64 ? k0 : k1;
      const uint64_t v = i < n_live ? pack_wi(idx, __uint_as_float(~hi[q])) : 0ull;
      if (i < k) out[i] = v;
    }
  }

  // select_top_k for CELLS <= 2 (one cell per physical lane).  The merge
  // emits the live slots in (weight descending, slot ascending) order: a
  // logical lane's cells leave the selection sort in (weight descending, cell
  // ascending) order, as it swaps on a strictly larger weight only, and the
  // merge takes equal head weights from the smaller logical lane first, so
  // equal weights come out by (L, c), that is by slot s = L*CELLS + c.  One
  // bitonic network over the wave sorts the keys (~weight bits, s) ascending
  // and lane i writes output entry i: a fixed number of steps per row instead
  // of a wave maximum per emitted entry.
  __device__ __forceinline__ void select_top_k_sorted(int32_t k, uint64_t *out) {
    static_assert(CELLS <= 2, "one cell per physical lane");
    const int lane = lane_id();
    // Slot `lane` into this lane: CELLS == 2 keeps slot s in physical lane
    // (s >> 1) + 32*(s & 1); CELLS == 1 keeps it in lane s < 32.
    int32_t sk = key[0];
    float sw = wt[0];
    if constexpr (CELLS == 2) {
      const int src = (lane >> 1) | ((lane & 1) << 5);
      sk = __shfl(sk, src, kWave);
      sw = __shfl(sw, src, kWave);
    } else {
      if (lane >= 32) sk = -1;
    }
    const bool live = sk != -1;
    const uint64_t lm = ballot(live);
    const int n_live = __popcll(lm);
    // Empty slots sort last.  Live slots are a prefix (slots fill in order and
    // never empty again), so after the stages up to the first block size that
    // covers the highest live slot, lanes [0, n_live) hold the live keys in
    // order; the later stages would only move the empty ones.
    uint32_t hi = live ? ~__float_as_uint(sw) : 0xFFFFFFFFu;
    uint32_t lo = live ? static_cast<uint32_t>(lane) : 0xFFFFFFFFu;
    const int span = lm ? 64 - __builtin_clzll(lm) : 0;
    bitonic_sort_prefix64<(CELLS == 2 ? 64 : 32)>(hi, lo, span);
    const int32_t idx = __shfl(sk, static_cast<int>(lo & 63u), kWave);
    const uint64_t v = lane < n_live ? pack_wi(idx, __uint_as_float(~hi)) : 0ull;
    if (lane < k) out[lane] = v;
  }
};

} // namespace sporder_hip
