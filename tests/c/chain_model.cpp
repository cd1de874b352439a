// chain_model.cpp -- host model of the compact chain walk of
// greedy_compact_kernel (chunkedgreedy_amd/csrc/csg.hip), lane by lane.
//
// Test infrastructure only (loaded by tests/test_chain_model.py).  The walk
// runs on one wave64; here its 64 lanes are arrays and every cross-lane
// operation follows the hardware rule the kernel depends on:
//   - ballot sees only active lanes;
//   - readlane / readfirstlane read a lane whatever the execution mask;
//   - a shuffle (ds_bpermute) returns 0 to an active lane whose source lane
//     is inactive (or, with inactive_zero = 0, the source's value: a machine
//     on which the mask did not matter).
// The LDS arrays have the kernel's layout sizes and are bounds-checked: an
// index outside its array is counted and reads 0.  Order writes outside the
// chunk are counted and not performed; a row written at a second position is
// counted.
//
// Staging modelled: 64-bit entries (weight bits, local index) sorted into
// preference order when a chunk's in-chunk entries fit entry_cap; else, when
// packed_cap > 0 and they fit the launch's packed capacity, 16-bit local
// indices in table order with each run of equal weight sorted by index (the
// kernel's packed rows, which need the table rows in weight order to give the
// same preference order); else table reads.  With packed_cap > 0 the chain
// is split over two launches as the host does it: the narrow launch packs up
// to min(packed_cap, 4 * entry_cap) entries, the second takes the chunks whose
// valid-entry sum S lies in (max(entry_cap, that), packed_cap] and packs up to
// packed_cap.
//
// Walks modelled:
//   variant 0: the kernel's walk, its mode chosen as the kernel chooses it
//              (table reads when the slice is neither staged nor packed, else
//              the one-entry mode when at least half the rows with entries
//              have exactly one, else the sorted scan with read-ahead, whose
//              steps over rows of at most 64 entries are the assembly block's
//              when the chunk has at most 64 bitmap words);
//   variants 1, 2, 3: the kernel's table, one-entry and sorted modes forced
//              (1 only applies to a slice past entry_cap, 2 and 3 to a
//              compacted one);
//   variant 10: a removed variant: per-row first entry in an int16 array,
//              then a scan of the row's other entries, and a restart search
//              over a rows-with-entries bitmap; its visited test ran the
//              bitmap shuffles only in the lanes that held a candidate
//              (`cl >= 0 && !visited(cl)`), and its walk loop had no bound.
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <vector>

namespace {

constexpr int W = 64;
constexpr int kOffBits = 15;
constexpr int32_t kOffMask = (1 << kOffBits) - 1;
constexpr int kSortedRow = 64;      // variant 10: rows longer than this stay unsorted
constexpr int16_t kUnsortedRow = -2;

struct Diag {
  int64_t overrun = 0;  // order writes outside [start, end)
  int64_t revisit = 0;  // rows written at a second position
  int64_t oob = 0;      // LDS indices outside their arrays
  int64_t misread = 0;  // shuffles from an inactive lane whose value was not 0
  int64_t runaway = 0;  // walks stopped by the model's step cap
  int64_t steps = 0;
  int64_t asm_exits[4] = {0, 0, 0, 0}; // assembly block returns: end, restart, long row, ring
};

inline int32_t wi_index(uint64_t v) { return static_cast<int32_t>(static_cast<uint32_t>(v)) - 1; }
inline float wi_weight(uint64_t v) {
  const uint32_t b = static_cast<uint32_t>(v >> 32);
  float f;
  std::memcpy(&f, &b, 4);
  return f;
}
inline int ctz64(uint64_t m) { return __builtin_ctzll(m); }

template <typename T> struct Checked {
  std::vector<T> a;
  Diag *d;
  T get(int64_t i) const {
    if (i < 0 || i >= static_cast<int64_t>(a.size())) {
      d->oob += 1;
      return T(0);
    }
    return a[static_cast<size_t>(i)];
  }
};

struct Wave {
  bool inactive_zero;
  Diag *d;
  // Shuffle: lane i (active in exec) reads src[idx[i] & 63].
  void shfl(const uint32_t *src, const int32_t *idx, uint64_t exec, uint32_t *out) const {
    for (int i = 0; i < W; ++i) {
      if (!((exec >> i) & 1)) continue;
      const int s = idx[i] & (W - 1);
      if ((exec >> s) & 1) {
        out[i] = src[s];
      } else {
        if (src[s] != 0) d->misread += 1;
        out[i] = inactive_zero ? 0u : src[s];
      }
    }
  }
  static uint64_t ballot(const bool *p, uint64_t exec) {
    uint64_t m = 0;
    for (int i = 0; i < W; ++i)
      if (((exec >> i) & 1) && p[i]) m |= 1ull << i;
    return m;
  }
};

struct Chunk {
  int32_t start, end, size, words;
  std::vector<std::vector<uint64_t>> rows; // in-chunk entries per row, preference order
  std::vector<std::vector<uint16_t>> packed; // the kernel's packed rows (16-bit local indices)
  std::vector<int32_t> in_count;
  int64_t total;
  int64_t valid; // S: valid entries of the slice (the sketch's per-row counts, summed)
};

// Staged entries as the kernel builds them: a row's in-chunk entries among its
// valid prefix, as (weight bits << 32) | local, in chain preference order
// (weight descending, local ascending).
Chunk stage(int32_t n, int32_t k, int32_t chunk_size, int64_t chunk, const uint64_t *table) {
  Chunk c;
  c.start = static_cast<int32_t>(chunk * chunk_size);
  c.end = static_cast<int32_t>(std::min<int64_t>(c.start + static_cast<int64_t>(chunk_size), n));
  c.size = c.end - c.start;
  c.words = (c.size + 31) >> 5;
  c.rows.assign(c.size, {});
  c.packed.assign(c.size, {});
  c.in_count.assign(c.size, 0);
  c.total = 0;
  c.valid = 0;
  for (int32_t r = 0; r < c.size; ++r) {
    const uint64_t *row = table + static_cast<size_t>(c.start + r) * k;
    // Valid entries form a prefix of the row (the sketch's count).
    int32_t rv = 0;
    while (rv < k && wi_index(row[rv]) >= 0) ++rv;
    c.valid += rv;
    for (int32_t j = 0; j < k; ++j) {
      const int32_t x = wi_index(row[j]);
      if (x < 0) continue;
      if (x >= c.start && x < c.end) {
        c.rows[r].push_back((row[j] & 0xFFFFFFFF00000000ull) | static_cast<uint32_t>(x - c.start));
      }
    }
    // Packed row as the kernel builds it: the valid prefix in table order,
    // in-chunk entries only; a run of equal weight bits starts wherever an
    // in-chunk entry's weight differs from the previous in-chunk entry's; each
    // run sorted by local index (insertion sort).
    std::vector<uint16_t> &pk = c.packed[r];
    std::vector<uint8_t> run_start;
    uint32_t prev_w = 0u;
    for (int32_t j = 0; j < rv; ++j) {
      const int32_t x = wi_index(row[j]);
      if (x < c.start || x >= c.end) continue;
      const uint32_t wb = static_cast<uint32_t>(row[j] >> 32);
      run_start.push_back(wb != prev_w);
      prev_w = wb;
      pk.push_back(static_cast<uint16_t>(x - c.start));
    }
    size_t rs = 0;
    for (size_t i = 1; i < pk.size(); ++i) {
      if (run_start[i]) {
        rs = i;
        continue;
      }
      const uint16_t v = pk[i];
      size_t j = i;
      while (j > rs && pk[j - 1] > v) {
        pk[j] = pk[j - 1];
        --j;
      }
      pk[j] = v;
    }
    std::sort(c.rows[r].begin(), c.rows[r].end(), [](uint64_t a, uint64_t b) {
      return (a ^ 0xFFFFFFFFull) > (b ^ 0xFFFFFFFFull);
    });
    c.in_count[r] = static_cast<int32_t>(c.rows[r].size());
    c.total += c.in_count[r];
  }
  return c;
}

struct Out {
  int32_t *order;
  std::vector<uint8_t> *seen; // rows already written
  Diag *d;
  const Chunk *c;
  void put(int64_t at, int32_t local) {
    uint8_t &s = (*seen)[static_cast<size_t>(c->start + local)];
    if (s) d->revisit += 1;
    s = 1;
    if (at < c->start || at >= c->end) {
      d->overrun += 1;
      return;
    }
    order[at] = c->start + local;
  }
};

// The kernel's walk (csg.hip, `walk`), modes 0 table, 1 single, 2 ahead.
// 64-bit words of the kernel's entries region (greedy_entry_words).
int32_t entry_words(int32_t entry_cap, int32_t packed_cap) {
  return entry_cap > (packed_cap + 3) / 4 ? entry_cap : (packed_cap + 3) / 4;
}

void walk_kernel(const Chunk &c, int mode, bool packed, int32_t k, int32_t rows_cap,
                 int32_t entry_cap, int32_t packed_cap, const uint64_t *table, Wave &wv,
                 Out &out, Diag &d) {
  const bool sorted = mode != 0, single = mode == 1, ahead = mode == 2;
  // LDS: entries u64[entry_words] (or 16-bit ones in the same bytes) |
  // offsets (row headers when sorted) i32[rows_cap + 1].
  const int32_t words64 = entry_words(entry_cap, packed_cap);
  Checked<uint64_t> ent{std::vector<uint64_t>(packed ? 0 : words64, 0), &d};
  Checked<uint16_t> ent16{std::vector<uint16_t>(packed ? 4 * static_cast<size_t>(words64) : 0, 0),
                          &d};
  Checked<int32_t> off{std::vector<int32_t>(rows_cap + 1, 0), &d};
  {
    int64_t a = 0;
    for (int32_t r = 0; r < c.size; ++r) {
      off.a[r] = static_cast<int32_t>(a);
      if (sorted && packed) {
        for (size_t j = 0; j < c.packed[r].size(); ++j) {
          if (a + static_cast<int64_t>(j) < static_cast<int64_t>(ent16.a.size())) {
            ent16.a[a + j] = c.packed[r][j];
          } else {
            d.oob += 1;
          }
        }
      } else if (sorted) {
        for (size_t j = 0; j < c.rows[r].size(); ++j) ent.a[a + j] = c.rows[r][j];
      }
      a += c.in_count[r];
    }
    off.a[c.size] = static_cast<int32_t>(a);
    if (sorted) {
      for (int32_t r = 0; r < c.size; ++r) {
        const int32_t a0 = off.a[r], b0 = off.a[r + 1] & kOffMask;
        const int32_t first = packed ? static_cast<int32_t>(ent16.get(a0))
                                     : static_cast<int32_t>(ent.get(a0) & 0xFFFu);
        if (b0 > a0) off.a[r] = a0 | (first << kOffBits);
      }
    }
  }
  const uint64_t all = ~0ull;
  const uint32_t tail = (c.size & 31) ? ((1u << (c.size & 31)) - 1u) : 0xFFFFFFFFu;
  uint32_t bm0[W] = {}, bm1[W] = {};
  auto full_bits = [&](int32_t w) { return w == c.words - 1 ? tail : 0xFFFFFFFFu; };
  auto mark = [&](int32_t w, uint32_t bits) {
    for (int l = 0; l < W; ++l) {
      bm0[l] |= l == w ? bits : 0u;
      bm1[l] |= l + W == w ? bits : 0u;
    }
  };
  int32_t cur = 0, low_word = 0;
  int64_t pos = c.start;
  bool have_next = false;
  int32_t nd0 = 0, nd1 = 0;
  const int64_t cap = 4 * static_cast<int64_t>(c.size) + 64;
  int64_t steps = 0;
  // Read-ahead walks over at most 64 bitmap words run their steps in the
  // kernel's assembly block (ahead_steps): every lane active, lanes past the
  // row repeating its last entry, positions held in a ring and stored when
  // the block returns (at a row with no free entry or more than 64 entries,
  // a full ring, or pos = end).
  const bool asm_steps = ahead && c.words <= W;
  while (pos < c.end) {
    int st = -1; // 0 end, 1 restart, 2 long row, 3 full ring
    if (asm_steps) {
      if (!have_next) {
        nd0 = off.get(cur);
        nd1 = off.get(cur + 1);
      }
      int32_t ring[W];
      int rp = 0;
      while (true) {
        if (pos >= c.end) {
          st = 0;
          break;
        }
        if (rp == W) {
          st = 3;
          break;
        }
        if (++steps > cap) {
          d.runaway += 1;
          st = 0;
          break;
        }
        d.steps += 1;
        mark(cur >> 5, 1u << (cur & 31));
        ring[rp++] = cur;
        pos += 1;
        const int32_t a0 = nd0 & kOffMask, len = (nd1 & kOffMask) - a0;
        if (len < 1) {
          st = 1;
          break;
        }
        if (len > W) {
          st = 2;
          break;
        }
        int32_t cl[W], o0[W], o1[W], wi[W];
        for (int l = 0; l < W; ++l) {
          const int32_t j = std::min(l, len - 1);
          cl[l] = packed ? static_cast<int32_t>(ent16.get(a0 + j))
                         : static_cast<int32_t>(static_cast<uint32_t>(ent.get(a0 + j)));
          o0[l] = off.get(cl[l]);
          o1[l] = off.get(cl[l] + 1);
          wi[l] = (cl[l] >> 5) & (W - 1); // ds_bpermute lane: address (cl >> 3), bits 7:2
        }
        uint32_t word[W];
        wv.shfl(bm0, wi, all, word);
        bool p[W];
        for (int l = 0; l < W; ++l) p[l] = l < len && !((word[l] >> (cl[l] & 31)) & 1u);
        const uint64_t m = Wave::ballot(p, all);
        if (m == 0) {
          st = 1;
          break;
        }
        const int l = ctz64(m);
        cur = cl[l];
        nd0 = o0[l];
        nd1 = o1[l];
      }
      for (int i = 0; i < rp; ++i) out.put(pos - rp + i, ring[i]);
      d.asm_exits[st] += 1;
      have_next = true;
      if (st == 0) break;
      if (st == 3) continue;
    } else {
      if (++steps > cap) {
        d.runaway += 1;
        break;
      }
      d.steps += 1;
      mark(cur >> 5, 1u << (cur & 31));
      out.put(pos, cur);
      pos += 1;
    }
    int32_t h0, h1;
    if (ahead) {
      h0 = have_next ? nd0 : off.get(cur);
      h1 = have_next ? nd1 : off.get(cur + 1);
      have_next = false;
    } else {
      h0 = off.get(cur);
      h1 = off.get(cur + 1);
    }
    const int32_t d0 = sorted ? (h0 & kOffMask) : h0;
    const int32_t d1 = sorted ? (h1 & kOffMask) : h1;
    int32_t best_c = -1;
    if (d1 > d0 && st != 1) {
      const int32_t c0 = (h0 >> kOffBits) & 0xFFF;
      bool first_free = false;
      if (single) {
        const int32_t w0 = c0 >> 5;
        const uint32_t word0 = w0 < W ? bm0[w0] : bm1[w0 - W];
        first_free = c0 < c.size && !((word0 >> (c0 & 31)) & 1u);
      }
      if (single && (first_free || d1 - d0 == 1)) {
        if (first_free) best_c = c0;
      } else if (sorted) {
        const int32_t len = d1 - d0;
        for (int32_t j0 = 0; j0 < len && best_c < 0; j0 += W) {
          int32_t cl[W], o0[W], o1[W], wi[W];
          for (int l = 0; l < W; ++l) {
            const int32_t j = j0 + l;
            cl[l] = -1;
            o0[l] = o1[l] = 0;
            if (j < len) {
              if (packed) {
                cl[l] = static_cast<int32_t>(ent16.get(d0 + j));
              } else {
                const uint64_t e = ent.get(d0 + j);
                cl[l] = static_cast<int32_t>(static_cast<uint32_t>(e));
              }
              if (ahead) {
                o0[l] = off.get(cl[l]);
                o1[l] = off.get(cl[l] + 1);
              }
            }
            wi[l] = cl[l] >= 0 ? cl[l] >> 5 : 0;
          }
          uint32_t word[W], v1[W];
          wv.shfl(bm0, wi, all, word);
          if (c.words > W) {
            wv.shfl(bm1, wi, all, v1);
            for (int l = 0; l < W; ++l) word[l] = wi[l] < W ? word[l] : v1[l];
          }
          bool p[W];
          for (int l = 0; l < W; ++l) p[l] = cl[l] >= 0 && !((word[l] >> (cl[l] & 31)) & 1u);
          const uint64_t m = Wave::ballot(p, all);
          if (m != 0) {
            const int l = ctz64(m);
            best_c = cl[l];
            if (ahead) {
              nd0 = o0[l];
              nd1 = o1[l];
              have_next = true;
            }
          }
        }
      } else {
        bool open[W];
        float bw[W];
        int32_t bc[W];
        for (int l = 0; l < W; ++l) {
          open[l] = true;
          bw[l] = -1.0f;
          bc[l] = -1;
        }
        for (int32_t j0 = 0; j0 < k; j0 += W) {
          int32_t cl[W], wi[W];
          float w[W];
          for (int l = 0; l < W; ++l) {
            const int32_t j = j0 + l;
            cl[l] = -1;
            w[l] = 0.0f;
            if (j < k) {
              const uint64_t e = table[static_cast<size_t>(c.start + cur) * k + j];
              const int32_t x = wi_index(e);
              if (x < 0) open[l] = false;
              cl[l] = (open[l] && x >= c.start && x < c.end) ? x - c.start : -1;
              w[l] = wi_weight(e);
            }
            wi[l] = cl[l] >= 0 ? cl[l] >> 5 : 0;
          }
          uint32_t word[W], v1[W];
          wv.shfl(bm0, wi, all, word);
          if (c.words > W) {
            wv.shfl(bm1, wi, all, v1);
            for (int l = 0; l < W; ++l) word[l] = wi[l] < W ? word[l] : v1[l];
          }
          for (int l = 0; l < W; ++l) {
            const bool cand = cl[l] >= 0 && !((word[l] >> (cl[l] & 31)) & 1u);
            if (cand && (w[l] > bw[l] || (w[l] == bw[l] && cl[l] < bc[l]))) {
              bw[l] = w[l];
              bc[l] = cl[l];
            }
          }
          if (Wave::ballot(open, all) != all) break;
        }
        // Largest weight, ties to the smaller index (lanes without a
        // candidate hold (-1, -1) and lose to any candidate).
        int best_l = -1;
        for (int l = 0; l < W; ++l) {
          if (bc[l] < 0) continue;
          if (best_l < 0 || bw[l] > bw[best_l] || (bw[l] == bw[best_l] && bc[l] < bc[best_l])) {
            best_l = l;
          }
        }
        best_c = best_l < 0 ? -1 : bc[best_l];
      }
    }
    if (best_c >= 0) {
      cur = best_c;
      continue;
    }
    int32_t nxt = -1;
    while (true) {
      uint32_t f0[W], f1[W];
      bool p0[W], p1[W];
      for (int l = 0; l < W; ++l) {
        f0[l] = (l < c.words && l >= low_word) ? (~bm0[l] & full_bits(l)) : 0u;
        f1[l] = (W + l < c.words && W + l >= low_word) ? (~bm1[l] & full_bits(W + l)) : 0u;
        p0[l] = f0[l] != 0u;
        p1[l] = f1[l] != 0u;
      }
      const uint64_t m0 = Wave::ballot(p0, all), m1 = Wave::ballot(p1, all);
      int32_t w = -1;
      uint32_t free_bits = 0u;
      if (m0 != 0) {
        w = ctz64(m0);
        free_bits = f0[w];
      } else if (m1 != 0) {
        w = W + ctz64(m1);
        free_bits = f1[w - W];
      }
      if (w < 0) break;
      low_word = w;
      bool has[W];
      for (int l = 0; l < W; ++l) {
        const int32_t r = w * 32 + (l & 31);
        const bool free_here = l < 32 && ((free_bits >> (l & 31)) & 1u);
        if (c.words <= W) {
          // The assembly search (restart_search): every lane reads the
          // headers of its row, clamped to the chunk's last row.
          const int32_t rc = std::min(r, c.size - 1);
          const int32_t a0 = off.get(rc), a1 = off.get(rc + 1);
          has[l] = free_here && (sorted ? (a1 & kOffMask) > (a0 & kOffMask) : a1 > a0);
        } else {
          has[l] = free_here && (sorted ? (off.get(r + 1) & kOffMask) > (off.get(r) & kOffMask)
                                        : off.get(r + 1) > off.get(r));
        }
      }
      const uint32_t with_entries = static_cast<uint32_t>(Wave::ballot(has, all));
      const uint32_t emit =
          with_entries ? free_bits & ((with_entries & (0u - with_entries)) - 1u) : free_bits;
      if (emit) {
        for (int l = 0; l < 32; ++l) {
          if ((emit >> l) & 1u) {
            const int64_t at = pos + __builtin_popcount(emit & ((1u << l) - 1u));
            if (at < c.end) out.put(at, w * 32 + l);
          }
        }
        mark(w, emit);
        pos += __builtin_popcount(emit);
      }
      if (with_entries) {
        nxt = w * 32 + __builtin_ctz(with_entries);
        break;
      }
    }
    if (nxt < 0) break;
    cur = nxt;
  }
}

// The removed variant's walk (compact slices only).
void walk_variant(const Chunk &c, int32_t k, int32_t rows_cap, int32_t entry_cap, bool compact,
                  const uint64_t *table, Wave &wv, Out &out, Diag &d) {
  Checked<uint64_t> ent{std::vector<uint64_t>(entry_cap, 0), &d};
  Checked<int32_t> off{std::vector<int32_t>(rows_cap + 1, 0), &d};
  Checked<int16_t> first{std::vector<int16_t>(rows_cap, -1), &d};
  std::vector<uint32_t> has_bm((rows_cap + 31) / 32, 0u);
  {
    int64_t a = 0;
    for (int32_t r = 0; r < c.size; ++r) {
      off.a[r] = static_cast<int32_t>(a);
      if (compact) {
        std::vector<uint64_t> row = c.rows[r];
        if (static_cast<int>(row.size()) > kSortedRow) {
          first.a[r] = kUnsortedRow; // left in table order for the arg-max scan
        } else {
          first.a[r] = row.empty() ? -1 : static_cast<int16_t>(static_cast<uint32_t>(row[0]));
        }
        for (size_t j = 0; j < row.size(); ++j) ent.a[a + j] = row[j];
      }
      if (c.in_count[r] > 0) has_bm[r >> 5] |= 1u << (r & 31);
      a += c.in_count[r];
    }
    off.a[c.size] = static_cast<int32_t>(a);
  }
  const uint64_t all = ~0ull;
  const uint32_t tail = (c.size & 31) ? ((1u << (c.size & 31)) - 1u) : 0xFFFFFFFFu;
  uint32_t bm0[W] = {}, bm1[W] = {}, has0[W] = {}, has1[W] = {};
  for (int l = 0; l < W; ++l) {
    has0[l] = l < c.words ? has_bm[l] : 0u;
    has1[l] = W + l < c.words ? has_bm[W + l] : 0u;
  }
  auto full_bits = [&](int32_t w) { return w == c.words - 1 ? tail : 0xFFFFFFFFu; };
  auto mark = [&](int32_t w, uint32_t bits) {
    for (int l = 0; l < W; ++l) {
      bm0[l] |= l == w ? bits : 0u;
      bm1[l] |= l + W == w ? bits : 0u;
    }
  };
  auto word_of = [&](const uint32_t *b0, const uint32_t *b1, int32_t w) {
    return w < W ? b0[w & (W - 1)] : b1[(w - W) & (W - 1)];
  };
  // visited_word under the mask `exec` (the lanes that evaluate it).
  auto visited_words = [&](const int32_t *cl, uint64_t exec, uint32_t *word) {
    int32_t wi[W];
    for (int l = 0; l < W; ++l) wi[l] = cl[l] >= 0 ? cl[l] >> 5 : 0;
    wv.shfl(bm0, wi, exec, word);
    if (c.words > W) {
      uint32_t v1[W];
      wv.shfl(bm1, wi, exec, v1);
      for (int l = 0; l < W; ++l)
        if ((exec >> l) & 1) word[l] = wi[l] < W ? word[l] : v1[l];
    }
  };
  int32_t cur = 0, low_word = 0;
  int64_t pos = c.start;
  const int64_t cap = 4 * static_cast<int64_t>(c.size) + 64;
  int64_t steps = 0;
  while (true) {
    if (++steps > cap) {
      d.runaway += 1;
      break;
    }
    d.steps += 1;
    mark(cur >> 5, 1u << (cur & 31));
    out.put(pos, cur);
    pos += 1;
    int32_t best_c = -1;
    auto scan_argmax = [&](bool from_lds, int32_t d0, int32_t len) {
      bool open[W];
      float bw[W];
      int32_t bc[W];
      for (int l = 0; l < W; ++l) {
        open[l] = true;
        bw[l] = -1.0f;
        bc[l] = -1;
      }
      for (int32_t j0 = 0; j0 < len; j0 += W) {
        int32_t cl[W];
        float w[W];
        uint64_t exec = 0;
        for (int l = 0; l < W; ++l) {
          const int32_t j = j0 + l;
          cl[l] = -1;
          w[l] = 0.0f;
          if (j < len) {
            if (from_lds) {
              const uint64_t e = ent.get(d0 + j);
              cl[l] = static_cast<int32_t>(static_cast<uint32_t>(e));
              w[l] = wi_weight(e);
            } else {
              const uint64_t e = table[static_cast<size_t>(c.start + cur) * k + j];
              const int32_t x = wi_index(e);
              if (x < 0) open[l] = false;
              cl[l] = (open[l] && x >= c.start && x < c.end) ? x - c.start : -1;
              w[l] = wi_weight(e);
            }
          }
          if (cl[l] >= 0) exec |= 1ull << l; // `cl >= 0 && ...` evaluates the rest here only
        }
        uint32_t word[W] = {};
        visited_words(cl, exec, word);
        for (int l = 0; l < W; ++l) {
          const bool cand = cl[l] >= 0 && !((word[l] >> (cl[l] & 31)) & 1u);
          if (cand && (w[l] > bw[l] || (w[l] == bw[l] && cl[l] < bc[l]))) {
            bw[l] = w[l];
            bc[l] = cl[l];
          }
        }
        if (!from_lds && Wave::ballot(open, all) != all) break;
      }
      int best_l = -1;
      for (int l = 0; l < W; ++l) {
        if (bc[l] < 0) continue;
        if (best_l < 0 || bw[l] > bw[best_l] || (bw[l] == bw[best_l] && bc[l] < bc[best_l])) {
          best_l = l;
        }
      }
      best_c = best_l < 0 ? -1 : bc[best_l];
    };
    if (compact) {
      const int32_t f = first.get(cur);
      if (f >= 0) {
        if (!((word_of(bm0, bm1, f >> 5) >> (f & 31)) & 1u)) {
          best_c = f;
        } else {
          const int32_t d0 = off.get(cur), len = off.get(cur + 1) - d0;
          for (int32_t j0 = 1; j0 < len; j0 += W) {
            int32_t cl[W];
            uint64_t exec = 0;
            for (int l = 0; l < W; ++l) {
              const int32_t j = j0 + l;
              const uint64_t e = j < len ? ent.get(d0 + j) : 0;
              cl[l] = j < len ? static_cast<int32_t>(static_cast<uint32_t>(e)) : -1;
              if (cl[l] >= 0) exec |= 1ull << l;
            }
            uint32_t word[W] = {};
            visited_words(cl, exec, word);
            bool p[W];
            for (int l = 0; l < W; ++l) p[l] = cl[l] >= 0 && !((word[l] >> (cl[l] & 31)) & 1u);
            const uint64_t m = Wave::ballot(p, all);
            if (m != 0) {
              best_c = cl[ctz64(m)];
              break;
            }
          }
        }
      } else if (f == kUnsortedRow) {
        const int32_t d0 = off.get(cur);
        scan_argmax(true, d0, off.get(cur + 1) - d0);
      }
    } else if (off.get(cur + 1) > off.get(cur)) {
      scan_argmax(false, 0, k);
    }
    if (best_c >= 0) {
      cur = best_c;
      continue;
    }
    int32_t nxt = -1;
    while (true) {
      uint32_t f0[W], f1[W];
      bool p0[W], p1[W];
      for (int l = 0; l < W; ++l) {
        f0[l] = (l < c.words && l >= low_word) ? (~bm0[l] & full_bits(l)) : 0u;
        f1[l] = (W + l < c.words && W + l >= low_word) ? (~bm1[l] & full_bits(W + l)) : 0u;
        p0[l] = f0[l] != 0u;
        p1[l] = f1[l] != 0u;
      }
      const uint64_t m0 = Wave::ballot(p0, all), m1 = Wave::ballot(p1, all);
      int32_t w = -1;
      uint32_t free_bits = 0u;
      if (m0 != 0) {
        w = ctz64(m0);
        free_bits = f0[w];
      } else if (m1 != 0) {
        w = W + ctz64(m1);
        free_bits = f1[w - W];
      }
      if (w < 0) break;
      low_word = w;
      const uint32_t with_entries = free_bits & word_of(has0, has1, w);
      const uint32_t emit =
          with_entries ? free_bits & ((with_entries & (0u - with_entries)) - 1u) : free_bits;
      if (emit) {
        for (int l = 0; l < 32; ++l) {
          if ((emit >> l) & 1u) out.put(pos + __builtin_popcount(emit & ((1u << l) - 1u)), w * 32 + l);
        }
        mark(w, emit);
        pos += __builtin_popcount(emit);
      }
      if (with_entries) {
        nxt = w * 32 + __builtin_ctz(with_entries);
        break;
      }
    }
    if (nxt < 0) break;
    cur = nxt;
  }
}

} // namespace

extern "C" {

// Runs the modelled walk over every chunk of `table` (n rows of k packed
// entries).  `order` receives the permutation (positions a walk did not
// write keep their previous value); diag[0..9] = overrun, revisit, oob,
// misread, runaway, steps, and the assembly step block's returns at pos = end,
// for a restart, at a row of more than 64 entries and at a full ring; mode_counts[0..5] = chunks walked in table,
// one-entry and sorted mode (variant 0), of those in a 16-bit packed form
// (one-entry, sorted), and chunks taken by the second launch.  packed_cap 0:
// no packed form and one launch (the wide launch, or statistics asked for).
// Returns 0, or -1 for a variant that does not apply to some chunk.
int32_t chain_model(int32_t n, int32_t k, int32_t chunk_size, const uint64_t *table,
                    int32_t entry_cap, int32_t packed_cap, int32_t variant,
                    int32_t inactive_zero, int32_t *order, int64_t *diag,
                    int64_t *mode_counts) {
  Diag d;
  std::vector<uint8_t> seen(static_cast<size_t>(n), 0);
  const int32_t rows_cap = std::min(chunk_size, n);
  Wave wv{inactive_zero != 0, &d};
  const int64_t chunks = (static_cast<int64_t>(n) + chunk_size - 1) / chunk_size;
  // The host's split (csg.hip, the narrow launch and the packed launch).
  const int32_t narrow_packed = std::min(packed_cap, 4 * entry_cap);
  const bool split = packed_cap > narrow_packed;
  const int64_t band_lo = std::max(entry_cap, narrow_packed);
  const int64_t band_hi = split ? packed_cap : 0;
  for (int64_t q = 0; q < chunks; ++q) {
    const Chunk c = stage(n, k, chunk_size, q, table);
    Out out{order, &seen, &d, &c};
    const bool second = split && band_lo < c.valid && c.valid <= band_hi;
    const int32_t launch_packed = second ? packed_cap : narrow_packed;
    mode_counts[5] += second;
    const bool compact = c.total <= entry_cap;
    const bool packed = !compact && c.total <= launch_packed;
    int single_rows = 0, entry_rows = 0;
    for (int32_t r = 0; r < c.size; ++r) {
      single_rows += c.in_count[r] == 1;
      entry_rows += c.in_count[r] > 0;
    }
    const bool staged = compact || packed;
    int mode;
    if (variant == 0) {
      mode = !staged ? 0 : (2 * single_rows >= entry_rows ? 1 : 2);
    } else if (variant >= 1 && variant <= 3) {
      mode = variant - 1;
      if ((mode == 0) == staged) return -1;
    } else if (variant == 10) {
      walk_variant(c, k, rows_cap, entry_cap, compact, table, wv, out, d);
      continue;
    } else {
      return -1;
    }
    mode_counts[mode] += 1;
    if (packed && mode != 0) mode_counts[mode + 2] += 1;
    walk_kernel(c, mode, packed, k, rows_cap, entry_cap, second ? packed_cap : narrow_packed,
                table, wv, out, d);
  }
  diag[0] = d.overrun;
  diag[1] = d.revisit;
  diag[2] = d.oob;
  diag[3] = d.misread;
  diag[4] = d.runaway;
  diag[5] = d.steps;
  for (int i = 0; i < 4; ++i) diag[6 + i] = d.asm_exits[i];
  return 0;
}

} // extern "C"
