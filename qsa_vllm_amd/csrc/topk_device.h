// Device side of the exact per-row top-k selection + token expansion.
//
// Semantics follow ops/csrc/topk.cu of the reference plugin:
//  * order key = raw fp32 bit pattern read as uint32 (topk.cu:262, 331-338),
//    larger key first, lower id first among equal keys;
//  * rows with length <= k emit ids 0..length-1 then -1 (topk.cu:187-191);
//  * selected ids are emitted in ascending id order (topk.cu:328-349);
//  * expansion, causal tail, physical slot mapping and counts as
//    ExpandedWriter (topk.cu:97-180).
//
// Algorithm (own design for wave64 + LDS). One workgroup per row loads the
// row coalesced (thread t holds elements i * THREADS + t). Each full wave
// bounds the m-th largest of its threads' maxima from below (m * full waves
// >= k); keys under the smallest bound cannot be selected. A whole row
// compacts the keys at or above the bound, in id order, straight from that
// layout (process_row_whole); a row with too many of them, or a part of a
// row, is staged through LDS so thread t owns ids [t*ITEMS, t*ITEMS+ITEMS)
// and pruned the same way (process_row). A radix select walks
// 8-bit digits downward from the highest bit in which the remaining keys
// differ (one block min/max). Each pass builds an LDS histogram
// (atomics with a wave-uniform fast path); after one barrier every wave reads
// it and locates the bin holding the k-th largest key with a DPP scan. The walk stops as soon as that bin
// holds exactly the number of keys still needed - then the selection is every
// key >= the bin's smallest possible key - or when all 32 bits are fixed, in
// which case the remaining slots go to the lowest ids with that exact key.
// A block-wide exclusive scan of (selected, tied) counts in id order gives
// each selected id its output rank; ranks land in LDS and the whole output row
// (expanded slots, causal tail, -1 padding) is written with coalesced stores.
//
// The kernel is a chain of short dependent steps, so latency is what counts:
// every independent load (scores, row metadata, the page-table entry of every
// block a thread holds, the causal tail's pages) is issued at entry, the
// barriers order LDS only (so those loads stay in flight through the radix
// passes), derived row metadata is computed only when the row is written, and
// reductions and scans are DPP sequences.
//
// A decode batch's rows (few, so latency counts) size the workgroup's keys
// per thread by the row's own length, up to 16384 keys at once; a row of up
// to 32768 keys takes its halves in turn and then the halves' winners, in one
// workgroup. Longer rows use two launches: exact top-k per 8192-column
// partition, then exact top-k over the partition winners. Fewer waves make
// each barrier-separated phase cheaper: a short row of a 1024-thread launch
// runs on its lower 512 threads from the start, and a 1024-thread row whose
// compacted candidates fit 1024 selects and writes on its lower 512 threads
// (the upper waves end; a barrier waits only for waves that have not ended).
#pragma once

#include "qsa_common.h"

extern "C" __device__ unsigned int __ockl_wfred_min_u32(unsigned int);
extern "C" __device__ unsigned int __ockl_wfred_max_u32(unsigned int);
extern "C" __device__ int __ockl_wfscan_add_i32(int, bool);

namespace qsa {
namespace {

constexpr int kPartitionColumns = 8192;
constexpr int kMaxDirectColumns = 16384;  // register-resident capacity: 1024 threads x 16 keys
constexpr int kMaxTopk = 8192;            // selected ids per row staged in LDS
constexpr int kTailSlots = 64;            // causal-tail pages fetched ahead of time

constexpr int kHistBuffers = 3;  // radix pass k counts into buffer k % 3
#ifndef QSA_TOPK_DIGIT_BITS
#define QSA_TOPK_DIGIT_BITS 8
#endif
constexpr int kDigitBits = QSA_TOPK_DIGIT_BITS;  // radix digit width
constexpr int kBins = 1 << kDigitBits;
constexpr int kBinsPerLane = kBins / 64;  // every wave scans the whole histogram
#ifndef QSA_TOPK_PRUNE
#define QSA_TOPK_PRUNE 1
#endif

template <int THREADS>
struct TopkShared {
  alignas(16) uint32_t hist[kHistBuffers][kBins];
  uint32_t wmin[THREADS / 64];
  uint32_t wmax[THREADS / 64];
  uint32_t wfloor[THREADS / 64];
  int wsel[THREADS / 64];
  int wtie[THREADS / 64];
  int tail_page[kTailSlots];
  int ccount[16 * (THREADS / 64)];  // whole-row path: candidates per (item, wave)
};

// --- row metadata -------------------------------------------------------------

struct ExpandMeta {
  const int64_t* positions;
  const int32_t* sequence_lengths;
  const int32_t* token_to_req;
  const int32_t* table;
  int32_t* counts;
  int64_t table_row_stride;
  int64_t out_col_stride;
  int num_requests;
  int table_width;
  int page_size;
  FastDiv page_div;
  int ratio;
  FastDiv ratio_div;
  int out_width;
  int physical;
  int store_counts;
};

// Expansion parameters of qsa_topk_expand's arguments (host side).
inline ExpandMeta make_expand_meta(const int64_t* positions, const int32_t* sequence_lengths,
                                   int num_requests, const int32_t* token_to_req,
                                   const int32_t* table, int64_t table_row_stride,
                                   int table_width, int32_t* counts, int64_t out_col_stride,
                                   int out_width, int ratio, int page_size, int physical,
                                   int store_counts) {
  ExpandMeta m = {};
  m.positions = positions;
  m.sequence_lengths = sequence_lengths;
  m.token_to_req = token_to_req;
  m.table = physical ? table : nullptr;
  m.counts = counts;
  m.table_row_stride = table_row_stride;
  m.out_col_stride = out_col_stride;
  m.num_requests = num_requests;
  m.table_width = physical ? table_width : 0;
  m.page_size = page_size > 0 ? page_size : 1;
  m.page_div = FastDiv::make(page_size > 0 ? page_size : 1);
  m.ratio = ratio;
  m.ratio_div = FastDiv::make(ratio);
  m.out_width = out_width;
  m.physical = physical ? 1 : 0;
  m.store_counts = store_counts ? 1 : 0;
  return m;
}

// Raw per-row inputs of the expansion (topk.cu:166-180); everything derived
// from them is computed when the row is written.
struct RowMeta {
  int seq_len;  // loaded per lane (see load_request); seq() is the row's value
  int pos;
  const int32_t* table_row;  // null unless physical
  __device__ __forceinline__ int seq() const { return __builtin_amdgcn_readfirstlane(seq_len); }
};

// Zero that the compiler cannot prove uniform. A load of a per-row value
// indexed with it is a vector load: it completes in order with the wave's
// other vector loads, whereas a scalar load shares its counter with LDS
// operations, so the first LDS wait after it would stall until it returned.
__device__ __forceinline__ int vector_zero() {
  int z = 0;
  asm volatile("" : "+v"(z));
  return z;
}

// x / ratio with C semantics: one multiply-high for x >= 0 (the integer
// division sequence runs only for a negative x).
__device__ __forceinline__ int div_ratio(const ExpandMeta& m, int x) {
  return x >= 0 ? m.ratio_div.div(x) : x / m.ratio;
}
// First token of the causal tail (the incomplete block) of position pos.
__device__ __forceinline__ int tail_start_of(const ExpandMeta& m, int pos) {
  return div_ratio(m, pos + 1) * m.ratio;
}

// Logical page of token t, or -1 when t has no page-table entry to read.
__device__ __forceinline__ int token_page(const ExpandMeta& m, int t) {
  if (t < 0) return -1;
  const int lp = m.page_div.div(t);
  return lp < m.table_width ? lp : -1;
}

// Physical slot of token t given its prefetched physical page (topk.cu:116-125).
__device__ __forceinline__ int slot_of(const ExpandMeta& m, const RowMeta& r, int t, int pp) {
  if (t < 0 || t >= r.seq()) return -1;
  if (!m.physical) return t;
  if (pp < 0) return -1;
  return pp * m.page_size + (t - m.page_div.div(t) * m.page_size);
}

__device__ __forceinline__ int table_entry(const RowMeta& r, int lp) {
  return (r.table_row && lp >= 0) ? r.table_row[lp] : -1;
}

// Physical slot of block id's first token given that token's page (-1: none).
__device__ __forceinline__ int first_slot(const ExpandMeta& m, int pp, int id) {
  const int first = id * m.ratio;
  return pp >= 0 ? pp * m.page_size + (first - m.page_div.div(first) * m.page_size) : -1;
}

// --- staging -----------------------------------------------------------------
//
// One row chunk of at most THREADS * ITEMS candidates passes through LDS.
// Element e is loaded by thread e % THREADS, so a wave-wide load reads 256
// consecutive bytes (a thread reading its own ITEMS consecutive words instead
// makes every load instruction touch ITEMS times as many cache lines), and is
// read back by thread e / ITEMS, which owns ITEMS consecutive ids as the
// selection and its id-ordered ranking need. With the expansion, the physical
// page of each element's first token is staged beside it and read back only
// for the selected elements.
//
// Every global load is unconditional: an element outside the row reads the
// zero block instead of being skipped. That keeps the number of loads a wave
// has in flight known at compile time, so waiting for the scores does not also
// wait for the page-table loads issued after them (a skipped, divergent load
// forces the compiler to drain every outstanding load instead).
template <int THREADS, int ITEMS, bool PAGES>
struct TopkStage {
  alignas(16) uint32_t key[THREADS * ITEMS];  // also holds sel[] once the keys are read back
  int page[PAGES ? THREADS * ITEMS : 1];
};

struct DirectLoader {  // ids start + i over a contiguous score row
  const float* scores;
  int start;
  __device__ __forceinline__ int id_at(int i) const { return start + i; }
};

struct IndirectLoader {  // candidate list of ids into a score row
  const float* scores;
  const int32_t* ids;
  __device__ __forceinline__ int id_at(int i) const { return ids[i]; }
};

// --- block primitives (DPP wave reductions/scans + one LDS exchange) --------

// A lower bound on the m-th largest (1 <= m <= 64) of the 64 lanes' values:
// radix descent with ballots over the kFloorBits bits below the lanes' common
// prefix; the bits under them stay zero, which can only lower the result.
// Every value is uniform across the wave.
#ifndef QSA_TOPK_FLOOR_BITS
#define QSA_TOPK_FLOOR_BITS 5
#endif
constexpr int kFloorBits = QSA_TOPK_FLOOR_BITS;
__device__ __forceinline__ uint32_t wave_floor_mth_largest(uint32_t v, int m) {
  const uint32_t vmax = __ockl_wfred_max_u32(v);
  const uint32_t vmin = __ockl_wfred_min_u32(v);
  if (vmax == vmin) return vmax;
  const int top = 31 - __builtin_clz(vmax ^ vmin);
  uint32_t value = top == 31 ? 0u : vmax & ~((2u << top) - 1u);
  uint64_t cand = ~0ull;  // lanes equal to `value` on the bits fixed so far
  int need = m;
#pragma unroll
  for (int i = 0; i < kFloorBits; ++i) {
    const int b = top - i;
    if (b < 0) break;
    const uint64_t ones = cand & __ballot((v >> b) & 1u);
    const int c = __builtin_popcountll(ones);
    if (c >= need) {
      cand = ones;
      value |= 1u << b;
    } else {
      cand &= ~ones;
      need -= c;
    }
  }
  return value;
}

// Block min, max and min of the per-wave floors, one barrier.
template <int THREADS>
__device__ __forceinline__ void block_bounds(uint32_t& lo, uint32_t& hi, uint32_t& floor,
                                             TopkShared<THREADS>& sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  lo = __ockl_wfred_min_u32(lo);
  hi = __ockl_wfred_max_u32(hi);
  if (lane == 0) {
    sh.wmin[wave] = lo;
    sh.wmax[wave] = hi;
    sh.wfloor[wave] = floor;
  }
  lds_barrier();
  lo = 0xffffffffu;
  hi = 0u;
  floor = 0xffffffffu;
#pragma unroll
  for (int w = 0; w < THREADS / 64; ++w) {
    lo = min(lo, sh.wmin[w]);
    hi = max(hi, sh.wmax[w]);
    floor = min(floor, sh.wfloor[w]);
  }
}

// Exclusive scan of two counters over threads in thread order.
template <int THREADS>
__device__ __forceinline__ void block_scan2(int& a, int& b, TopkShared<THREADS>& sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ea = __ockl_wfscan_add_i32(a, false);
  const int eb = __ockl_wfscan_add_i32(b, false);
  if (lane == 63) {
    sh.wsel[wave] = ea + a;
    sh.wtie[wave] = eb + b;
  }
  lds_barrier();
  int pa = 0, pb = 0;
#pragma unroll
  for (int w = 0; w < THREADS / 64; ++w) {
    if (w < wave) {
      pa += sh.wsel[w];
      pb += sh.wtie[w];
    }
  }
  a = pa + ea;
  b = pb + eb;
}

// --- selection --------------------------------------------------------------

// Exact top-k among the candidate keys (bit j of `cand`: key[j] is one) of
// a row whose candidates all lie in [lo, hi] and include every key that can
// be selected. Writes the selected ids in ascending-id order to sel[0..topk)
// and, with PAGES, the physical slot of each one's first token (from
// page[pos[j]], the staged page of the element) to sel[topk..2 topk).
// Candidates are in id order across threads (thread t's before thread t+1's).
//
// radix_rank_emit hands each selected candidate to emit(rank, id, pos)
// instead (rank: its place in ascending-id order).
template <int THREADS, int ITEMS, typename Emit>
__device__ __forceinline__ void radix_rank_emit(int topk, uint32_t lo, uint32_t hi, uint32_t cand,
                                                const uint32_t (&key)[ITEMS],
                                                const int (&id)[ITEMS], const int (&pos)[ITEMS],
                                                TopkShared<THREADS>& sh, Emit&& emit) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const uint32_t cand0 = cand;
  // Result: selected = {key > thr} + first `remaining` ids with key == thr
  // (tie mode), or {key >= thr} (ge mode).
  uint32_t thr = lo;
  bool ge = false;
  int remaining = topk;
  if (lo != hi) {
    constexpr uint32_t kDigitMask = kBins - 1;
    const int high_bit = 31 - __builtin_clz(lo ^ hi);
    int shift = high_bit > kDigitBits - 1 ? high_bit - (kDigitBits - 1) : 0;
    uint32_t prefix = shift + kDigitBits >= 32 ? 0u : (lo & ~((1u << (shift + kDigitBits)) - 1u));
    // One barrier per pass: every wave reads the whole histogram and finds
    // the bin itself (identical results), and pass k counts into buffer
    // k % 3, so the buffer read in pass k - 1 can be cleared during pass k
    // (all waves finished reading it before their pass-k atomics) and is
    // clean again by pass k + 2.
    for (int pass = 0;; ++pass) {
      uint32_t* hist = sh.hist[pass % kHistBuffers];
#pragma unroll
      for (int j = 0; j < ITEMS; ++j) {
        const bool a = (cand >> j) & 1u;
        const int d = (int)((key[j] >> shift) & kDigitMask);
        const uint64_t am = __ballot(a);
        if (am == 0) continue;
        const int first = __builtin_ctzll(am);
        const int d_first = __builtin_amdgcn_readlane(d, first);
        const uint64_t same = __ballot(a && d == d_first);
        if (same == am) {
          if (lane == first) atomicAdd(&hist[d], (uint32_t)__builtin_popcountll(am));
        } else if (a) {
          atomicAdd(&hist[d], 1u);
        }
      }
      lds_barrier();
      if (pass > 0 && tid < 64) {
        uint32_t* old = sh.hist[(pass - 1) % kHistBuffers] + kBinsPerLane * lane;
#pragma unroll
        for (int i = 0; i < kBinsPerLane; i += 4)
          *reinterpret_cast<u32x4*>(old + i) = u32x4{0u, 0u, 0u, 0u};
      }
      // Bin of the remaining-th largest candidate; lane owns kBinsPerLane
      // consecutive bins.
      uint32_t h[kBinsPerLane];
#pragma unroll
      for (int i = 0; i < kBinsPerLane; i += 4) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(hist + kBinsPerLane * lane + i);
        h[i] = v[0];
        h[i + 1] = v[1];
        h[i + 2] = v[2];
        h[i + 3] = v[3];
      }
      int tot = 0;
#pragma unroll
      for (int i = 0; i < kBinsPerLane; ++i) tot += (int)h[i];
      const int excl = __ockl_wfscan_add_i32(tot, false);
      const int total = __builtin_amdgcn_readlane(excl + tot, 63);
      int above = total - excl - tot;  // candidates in higher lanes' bins
      int hit = -1, hit_need = 0, hit_count = 0;
#pragma unroll
      for (int i = kBinsPerLane - 1; i >= 0; --i) {
        if (above < remaining && above + (int)h[i] >= remaining) {
          hit = kBinsPerLane * lane + i;
          hit_need = remaining - above;
          hit_count = (int)h[i];
        }
        above += (int)h[i];
      }
      const int src = __builtin_ctzll(__ballot(hit >= 0));
      const uint32_t bin = (uint32_t)__builtin_amdgcn_readlane(hit, src);
      const int need = __builtin_amdgcn_readlane(hit_need, src);
      const int in_bin = __builtin_amdgcn_readlane(hit_count, src);
      prefix |= bin << shift;
      if (in_bin == need) {  // the whole bin is taken: every candidate >= its smallest key
        thr = max(prefix, lo);
        ge = true;
        break;
      }
      uint32_t next = 0;
#pragma unroll
      for (int j = 0; j < ITEMS; ++j)
        if (((cand >> j) & 1u) && ((key[j] >> shift) & kDigitMask) == bin) next |= 1u << j;
      cand = next;
      remaining = need;
      if (shift == 0) {  // all 32 bits fixed: the bin holds one key value
        thr = prefix;
        break;
      }
      shift = shift >= kDigitBits ? shift - kDigitBits : 0;
    }
  }

  int n_sel = 0, n_tie = 0;
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    if ((cand0 >> j) & 1u) {
      n_sel += ge ? key[j] >= thr : key[j] > thr;
      n_tie += !ge && key[j] == thr;
    }
  }
  block_scan2<THREADS>(n_sel, n_tie, sh);
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    if (!((cand0 >> j) & 1u)) continue;
    const bool strict = ge ? key[j] >= thr : key[j] > thr;
    int rank = -1;
    if (strict) {
      rank = n_sel + min(n_tie, remaining);
      ++n_sel;
    } else if (!ge && key[j] == thr) {
      if (n_tie < remaining) rank = n_sel + n_tie;
      ++n_tie;
    }
    if (rank >= 0) emit(rank, id[j], pos[j]);
  }
}

template <int THREADS, int ITEMS, bool PAGES>
__device__ __forceinline__ void radix_rank(int topk, uint32_t lo, uint32_t hi, uint32_t cand,
                                           const uint32_t (&key)[ITEMS], const int (&id)[ITEMS],
                                           const int (&pos)[ITEMS], const int* page,
                                           const ExpandMeta& m, TopkShared<THREADS>& sh, int* sel) {
  radix_rank_emit<THREADS, ITEMS>(topk, lo, hi, cand, key, id, pos, sh,
                                  [&](int rank, int i, int p) {
                                    sel[rank] = i;
                                    sel[topk + rank] = PAGES ? first_slot(m, page[p], i) : -1;
                                  });
}

// Exact top-k of `length` (> topk) keys in registers (thread t holds
// elements t ITEMS .. t ITEMS + ITEMS - 1 of the row). Writes the selected ids
// in ascending-id order to sel[0..topk) and, with PAGES, the physical slot of
// each one's first token (from page[e], the staged page of the element at
// position e) to sel[topk..2 topk). `scratch` (scratch_words 32-bit words of
// LDS, dead until the selection is written) holds the compacted candidates.
template <int THREADS, int ITEMS, bool PAGES>
__device__ __forceinline__ void select_long(int length, int topk, const uint32_t (&key)[ITEMS],
                            const int (&id)[ITEMS], const int* page, const ExpandMeta& m,
                            TopkShared<THREADS>& sh, int* sel, uint32_t* scratch,
                            int scratch_words) {
  const int tid = threadIdx.x;
  const int base = tid * ITEMS;
  uint32_t active = 0;
  uint32_t lo = 0xffffffffu, hi = 0u;
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    if (base + j < length) {
      active |= 1u << j;
      lo = min(lo, key[j]);
      hi = max(hi, key[j]);
    }
  }
  // Lower bound on the topk-th largest key. Active threads are a prefix, so
  // waves [0, full) have 64 active lanes, each holding its thread maximum
  // (`hi` here, a distinct element). If each of those waves bounds the m-th
  // largest of its maxima from below, with m * full >= topk, at least topk
  // distinct elements are >= the smallest of these floors: keys below it
  // cannot be selected and never enter the histograms.
  uint32_t floor = 0u;  // 0: no bound
#if QSA_TOPK_PRUNE
  {
    const int threads_active = min(THREADS, (length + ITEMS - 1) / ITEMS);
    const int full = threads_active / 64;
    const int mm = full > 0 ? (topk + full - 1) / full : 65;
    if (mm <= 64) floor = (tid >> 6) < full ? wave_floor_mth_largest(hi, mm) : 0xffffffffu;
  }
#endif
  block_bounds<THREADS>(lo, hi, floor, sh);
  lo = max(lo, floor);  // smallest candidate bound; lo <= hi still holds
  uint32_t cand = 0;
#pragma unroll
  for (int j = 0; j < ITEMS; ++j)
    if (((active >> j) & 1u) && key[j] >= lo) cand |= 1u << j;

  if constexpr (ITEMS >= 4) {
    // Few candidates (the usual case once the bound has pruned): compact them,
    // in id order, to kCompact per thread and select among those, so the
    // radix passes and the ranking loop over kCompact keys per thread instead
    // of ITEMS. Three arrays of kCompact x THREADS words: keys, ids, positions.
    constexpr int kCompact = ITEMS >= 8 ? 2 : 1;
    int off = __builtin_popcount(cand), unused = 0;
    block_scan2<THREADS>(off, unused, sh);
    int total = 0;
#pragma unroll
    for (int w = 0; w < THREADS / 64; ++w) total += sh.wsel[w];
    if (total <= kCompact * THREADS && 3 * kCompact * THREADS <= scratch_words) {
      uint32_t* ckey = scratch;
      int* cid = reinterpret_cast<int*>(scratch + kCompact * THREADS);
      int* cpos = cid + kCompact * THREADS;
      int o = off;
#pragma unroll
      for (int j = 0; j < ITEMS; ++j) {
        if ((cand >> j) & 1u) {
          ckey[o] = key[j];
          cid[o] = id[j];
          cpos[o] = base + j;
          ++o;
        }
      }
      lds_barrier();
      uint32_t ck[kCompact];
      int ci[kCompact], cp[kCompact];
      uint32_t ccand = 0;
#pragma unroll
      for (int j = 0; j < kCompact; ++j) {
        const int e = kCompact * tid + j;
        const bool ok = e < total;
        ck[j] = ok ? ckey[e] : 0u;
        ci[j] = ok ? cid[e] : 0;
        cp[j] = ok ? cpos[e] : 0;
        ccand |= (uint32_t)ok << j;
      }
      // sel may share the scratch words: radix_rank writes it only after the
      // barrier of its rank scan, which every wave reaches with its
      // candidates already in registers, so no barrier is needed here.
      radix_rank<THREADS, kCompact, PAGES>(topk, lo, hi, ccand, ck, ci, cp, page, m, sh, sel);
      return;
    }
    lds_barrier();  // every wave has read the scan totals before they are reused
  }
  int pos[ITEMS];
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) pos[j] = base + j;
  radix_rank<THREADS, ITEMS, PAGES>(topk, lo, hi, cand, key, id, pos, page, m, sh, sel);
}

// Writes one expanded output row from ranked block ids in sel[0..topk) and
// the physical slots of their first tokens in sel[topk..) (-1 without one).
// Consecutive threads write consecutive columns.
//
// The common layouts (logical ids, or blocks that lie inside one page with the
// causal tail's pages prefetched) write the row from LDS alone, in a loop with
// no global load: on gfx9 stores count in the same in-order counter as loads,
// and the compiler cannot tell a skipped load from a pending one, so a load
// anywhere in the loop would make every iteration wait for all earlier stores.
// Tokens of an expanded row: the complete selected blocks (at most topk) and
// the causal tail, together at most the sequence length (the row's count).
struct ExpandedSpan {
  int expanded;    // complete blocks x ratio
  int tail_start;  // first token of the causal tail
  int tail_count;
  __device__ __forceinline__ int count(const RowMeta& r) const {
    return min(expanded + tail_count, r.seq());
  }
};
__device__ __forceinline__ ExpandedSpan expanded_span(const ExpandMeta& m, const RowMeta& r,
                                                      int topk) {
  const int p1 = r.pos + 1;
  const int complete = max(0, min(min(div_ratio(m, p1), div_ratio(m, r.seq())), topk));
  const int tail_start = tail_start_of(m, r.pos);
  return ExpandedSpan{complete * m.ratio, tail_start, p1 - tail_start};
}

__device__ __forceinline__ void write_expanded(const ExpandMeta& m, const RowMeta& r, int row,
                                               int topk, const int* sel, const int* tail_page,
                                               int32_t* out, int threads) {
  const ExpandedSpan span = expanded_span(m, r, topk);
  const int tail_start = span.tail_start;
  const int tail_count = span.tail_count;
  const int expanded = span.expanded;
  const bool block_in_page = m.physical && (m.page_size % m.ratio == 0);
  const bool from_lds = !m.physical || (block_in_page && m.ratio - 1 <= kTailSlots);
  const int64_t cs = m.out_col_stride;
  if (from_lds) {
    for (int c = threadIdx.x; c < m.out_width; c += threads) {
      int v = -1;
      if (c < expanded) {
        const int rank = m.ratio_div.div(c);
        const int o = c - rank * m.ratio;
        const int block = sel[rank];
        const int t = block * m.ratio + o;
        if (block >= 0 && t < r.seq()) {
          if (!m.physical) {
            v = t;
          } else {  // the block lies inside one page (topk.cu:134-146)
            const int s0 = sel[topk + rank];
            v = s0 >= 0 ? s0 + o : -1;
          }
        }
      } else {
        const int off = c - expanded;
        if (off < tail_count && off < m.ratio - 1)
          v = slot_of(m, r, tail_start + off, m.physical ? tail_page[off] : 0);
      }
      out[(int64_t)c * cs] = v;
    }
  } else {
    for (int c = threadIdx.x; c < m.out_width; c += threads) {
      int v = -1;
      if (c < expanded) {
        const int rank = m.ratio_div.div(c);
        const int o = c - rank * m.ratio;
        const int block = sel[rank];
        const int t = block * m.ratio + o;
        if (block >= 0 && t < r.seq()) {
          if (block_in_page) {
            const int s0 = sel[topk + rank];
            v = s0 >= 0 ? s0 + o : -1;
          } else {
            v = slot_of(m, r, t, table_entry(r, token_page(m, t)));
          }
        }
      } else {
        const int off = c - expanded;
        if (off < tail_count && off < m.ratio - 1) {
          const int t = tail_start + off;
          const int pp = off < kTailSlots ? tail_page[off] : table_entry(r, token_page(m, t));
          v = slot_of(m, r, t, pp);
        }
      }
      out[(int64_t)c * cs] = v;
    }
  }
  if (m.store_counts && threadIdx.x == 0) m.counts[row] = span.count(r);
}

// Row metadata and causal-tail pages of the expansion, loaded while the
// scores are in flight.
struct RowPrefetch {
  RowMeta r;
  int tail_pp;
  bool tail_ok;
};

// VSEQ loads the sequence length per lane (vector_zero), for callers that
// must not wait for it at their next LDS wait.
template <bool EXPAND, bool VSEQ = false>
__device__ __forceinline__ RowPrefetch prefetch_tail(const ExpandMeta& m, int req, int pos) {
  RowPrefetch f{RowMeta{0, pos, nullptr}, -1, false};
  if (!EXPAND) return f;
  const bool mapped = req >= 0 && req < m.num_requests;
  f.r.seq_len = mapped ? m.sequence_lengths[req + (VSEQ ? vector_zero() : 0)] : 0;
  f.r.table_row = m.physical ? m.table + (int64_t)(mapped ? req : 0) * m.table_row_stride : nullptr;
  const int tid = threadIdx.x;
  const int lp = (tid < kTailSlots && tid < m.ratio - 1) ? token_page(m, tail_start_of(m, pos) + tid)
                                                          : -1;
  f.tail_ok = f.r.table_row && lp >= 0;
  f.tail_pp = *(f.tail_ok ? f.r.table_row + lp : reinterpret_cast<const int32_t*>(g_qsa_zero_rows));
  return f;
}

// Physical page of block id's first token (-1 without one); unconditional load.
__device__ __forceinline__ int block_page(const ExpandMeta& m, const RowMeta& r, int id, bool in) {
  const int lp = in ? token_page(m, id * m.ratio) : -1;
  const bool ok = r.table_row && lp >= 0;
  return *(ok ? r.table_row + lp : g_qsa_no_page);
}

template <int THREADS>
__device__ __forceinline__ void clear_histograms(TopkShared<THREADS>& sh) {
  for (int b = threadIdx.x; b < kHistBuffers * kBins; b += THREADS) (&sh.hist[0][0])[b] = 0u;
}

// Scores of a contiguous row's elements [0, limit): element i * THREADS +
// tid's score in thread tid's v[i].
template <int THREADS, int ITEMS>
__device__ __forceinline__ void load_scores(const DirectLoader& load, int limit,
                                            uint32_t (&v)[ITEMS]) {
  const int tid = threadIdx.x;
  const uint32_t* src = reinterpret_cast<const uint32_t*>(load.scores + load.start);
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int e = i * THREADS + tid;
    v[i] = *(e < limit ? src + e : g_qsa_zero_rows);
  }
}

// Physical page of the first token of every element [0, limit) of a
// contiguous row (element i * THREADS + tid in pg[i], as load_scores), read
// from page-table row `table_row` (null: -1 everywhere).
template <int THREADS, int ITEMS>
__device__ __forceinline__ void load_element_pages(const DirectLoader& load, int limit,
                                                   const ExpandMeta& m,
                                                   const int32_t* table_row, int (&pg)[ITEMS]) {
  const RowMeta r{0, 0, table_row};
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int e = i * THREADS + threadIdx.x;
    pg[i] = block_page(m, r, load.start + e, e < limit);
  }
}

// The row's request and position, loaded per lane after the scores: a wave's
// vector loads complete in order, so the scores can be used while these are
// in flight, and no LDS wait stalls on them (vector_zero). The position is
// used as an int (its low word, little-endian): loading only that word keeps
// the load's whole destination live until it is used, so the compiler does
// not drain every load in flight to reuse a dead high half.
//
// With PAGES, the element pages are loaded at the same time from the table
// row of request `row` (clamped to the requests), the row's request in a
// decode batch of one-token requests, instead of after the request arrives;
// load_pages loads them again from the right row when the request differs.
struct RowRequest {
  int req;
  int pos;
  const int32_t* guess_row;  // table row of the pages in flight (null: none)
};
template <int THREADS, int ITEMS, bool EXPAND, bool PAGES>
__device__ __forceinline__ RowRequest load_request(const DirectLoader& load, int limit,
                                                   const ExpandMeta& m, int row,
                                                   int (&pg)[ITEMS]) {
  RowRequest q{0, 0, nullptr};
  if (!EXPAND) return q;
  // Unconditional (a null row reads -1 entries): loads issued under a branch
  // would leave the compiler unsure how many are in flight after it, and it
  // would then wait for these pages too before using the scores.
  if (PAGES) {
    if (m.table && m.num_requests > 0)
      q.guess_row = m.table + (int64_t)min(row, m.num_requests - 1) * m.table_row_stride;
    load_element_pages<THREADS, ITEMS>(load, limit, m, q.guess_row, pg);
  }
  const int z = vector_zero();
  const int32_t* pos_words = reinterpret_cast<const int32_t*>(m.positions);
  q.req = m.token_to_req[row + z];
  q.pos = pos_words[2 * (row + z)];
  return q;
}

// The expansion's row metadata and causal-tail pages, after the request
// arrives; with PAGES, the element pages again when the ones in flight came
// from another request's table row.
template <int THREADS, int ITEMS, bool EXPAND, bool PAGES>
__device__ __forceinline__ RowPrefetch load_pages(const DirectLoader& load, int limit,
                                                  const ExpandMeta& m, const RowRequest& q,
                                                  int (&pg)[ITEMS]) {
  const int req = __builtin_amdgcn_readfirstlane(q.req);
  const int pos = __builtin_amdgcn_readfirstlane(q.pos);
  const RowPrefetch f = prefetch_tail<EXPAND, true>(m, req, pos);
  if (PAGES && f.r.table_row != q.guess_row)  // uniform
    load_element_pages<THREADS, ITEMS>(load, limit, m, f.r.table_row, pg);
  return f;
}

// All the loads of a contiguous row: the row's request and position first
// (the tail and page loads depend on them, the scores do not), the scores,
// then the metadata and pages of the request.
template <int THREADS, int ITEMS, bool EXPAND, bool PAGES>
__device__ __forceinline__ RowPrefetch load_row(const DirectLoader& load, int limit,
                                                const ExpandMeta& m, int row, uint32_t (&v)[ITEMS],
                                                int (&pg)[ITEMS]) {
  const int req = EXPAND ? m.token_to_req[row] : 0;
  const int pos = EXPAND ? (int)m.positions[row] : 0;
  load_scores<THREADS, ITEMS>(load, limit, v);
  const RowPrefetch f = prefetch_tail<EXPAND>(m, req, pos);
  if (PAGES) load_element_pages<THREADS, ITEMS>(load, limit, m, f.r.table_row, pg);
  return f;
}

// The loaded scores (and pages) into the stage, then each thread's ITEMS
// consecutive keys back into registers. Ends with the barrier that also
// publishes the cleared histograms.
template <int THREADS, int ITEMS, bool PAGES, typename Stage>
__device__ __forceinline__ void stage_loaded(const DirectLoader& load, const uint32_t (&v)[ITEMS],
                                             const int (&pg)[ITEMS], uint32_t (&key)[ITEMS],
                                             int (&id)[ITEMS], TopkShared<THREADS>& sh, Stage& st) {
  const int tid = threadIdx.x;
  clear_histograms(sh);
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) st.key[i * THREADS + tid] = v[i];
  if (PAGES) {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) st.page[i * THREADS + tid] = pg[i];
  }
  lds_barrier();
  static_assert(ITEMS % 2 == 0, "keys are read back in pairs or quads");
#pragma unroll
  for (int j = 0; j < ITEMS; j += (ITEMS % 4 == 0 ? 4 : 2)) {
    if (ITEMS % 4 == 0) {
      const u32x4 q = *reinterpret_cast<const u32x4*>(&st.key[tid * ITEMS + j]);
      key[j] = q[0];
      key[j + 1] = q[1];
      key[j + 2] = q[2];
      key[j + 3] = q[3];
    } else {
      const u32x2 q = *reinterpret_cast<const u32x2*>(&st.key[tid * ITEMS + j]);
      key[j] = q[0];
      key[j + 1] = q[1];
    }
  }
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) id[j] = load.start + tid * ITEMS + j;
}

// Scores of elements [0, limit) of a contiguous row into the stage, then each
// thread's ITEMS consecutive keys back into registers.
template <int THREADS, int ITEMS, bool EXPAND, bool PAGES, typename Stage>
__device__ __forceinline__ RowPrefetch stage_row(const DirectLoader& load, int limit,
                                                 const ExpandMeta& m, int row, uint32_t (&key)[ITEMS],
                                                 int (&id)[ITEMS], TopkShared<THREADS>& sh, Stage& st) {
  uint32_t v[ITEMS];
  int pg[ITEMS];
  const RowPrefetch f = load_row<THREADS, ITEMS, EXPAND, PAGES>(load, limit, m, row, v, pg);
  stage_loaded<THREADS, ITEMS, PAGES>(load, v, pg, key, id, sh, st);
  return f;
}

// Candidate list: thread t gathers the ids at list positions [t*ITEMS,
// t*ITEMS+ITEMS) and their scores (and pages) directly.
template <int THREADS, int ITEMS, bool EXPAND, bool PAGES, typename Stage>
__device__ __forceinline__ RowPrefetch stage_row(const IndirectLoader& load, int limit,
                                                 const ExpandMeta& m, int row, uint32_t (&key)[ITEMS],
                                                 int (&id)[ITEMS], TopkShared<THREADS>& sh, Stage& st) {
  const int tid = threadIdx.x;
  const int base = tid * ITEMS;
  const int req = EXPAND ? m.token_to_req[row] : 0;
  const int pos = EXPAND ? (int)m.positions[row] : 0;
  const uint32_t* src = reinterpret_cast<const uint32_t*>(load.scores);
  const int32_t* zero = reinterpret_cast<const int32_t*>(g_qsa_zero_rows);
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) id[j] = *(base + j < limit ? load.ids + base + j : zero);
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) key[j] = src[id[j]];  // id 0 stands in past the list
  const RowPrefetch f = prefetch_tail<EXPAND>(m, req, pos);
  clear_histograms(sh);
  if (PAGES) {
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) st.page[base + j] = block_page(m, f.r, id[j], base + j < limit);
  }
  lds_barrier();
  return f;
}

// Writes the selected row (sel[0..topk) ranked ids, sel[topk..) their first
// slots) after the causal-tail pages are in LDS.
template <int THREADS, bool EXPAND>
__device__ __forceinline__ void write_row(const RowPrefetch& f, int topk, const ExpandMeta& m,
                                          int row, int32_t* out, TopkShared<THREADS>& sh,
                                          const int* sel) {
  const int tid = threadIdx.x;
  if (EXPAND && tid < kTailSlots && tid < m.ratio - 1) sh.tail_page[tid] = f.tail_ok ? f.tail_pp : -1;
  lds_barrier();
  if (EXPAND) {
    write_expanded(m, f.r, row, topk, sel, sh.tail_page, out, THREADS);
  } else {
    for (int c = tid; c < topk; c += THREADS) out[c] = sel[c];
  }
}

// Select and write one row from staged keys. `sel` (2 * topk ints) may alias
// the key stage, which is dead once the keys are in registers.
template <int THREADS, int ITEMS, bool EXPAND, bool PAGES, typename Loader, typename Stage>
__device__ __forceinline__ void finish_row(const Loader& load, const uint32_t (&key)[ITEMS],
                                           const int (&id)[ITEMS], const RowPrefetch& f,
                                           const Stage& st, int staged, int length_raw, int clamp,
                                           int topk, const ExpandMeta& m, int row, int32_t* out,
                                           TopkShared<THREADS>& sh, int* sel) {
  const int tid = threadIdx.x;
  const int length = length_raw > topk ? min(length_raw, clamp) : length_raw;
  if (length > topk) {
    select_long<THREADS, ITEMS, PAGES>(length, topk, key, id, st.page, m, sh, sel,
                                       reinterpret_cast<uint32_t*>(const_cast<uint32_t*>(st.key)),
                                       THREADS * ITEMS);
  } else {
    // At most topk entries: the loader's first `length` ids in order, then -1.
    lds_barrier();  // every wave has read its keys back before sel overwrites them
    // Lengths of at most topk are not clamped to the row, so ids past the
    // staged elements read their page directly.
    for (int i = tid; i < topk; i += THREADS) {
      const int lid = i < length ? load.id_at(i) : -1;
      sel[i] = lid;
      sel[topk + i] = (PAGES && lid >= 0)
                          ? first_slot(m, i < staged ? st.page[i] : block_page(m, f.r, lid, true), lid)
                          : -1;
    }
  }
  write_row<THREADS, EXPAND>(f, topk, m, row, out, sh, sel);
}

// One row: stage the scores (and pages), select, write. PAGES stages the
// physical page of every candidate (the expansion maps to physical slots); the
// stage must then have room for them.
//
// Everything down to here is force-inlined: a kernel that instantiates several
// row shapes would otherwise call them as functions, with their arguments
// and arrays in scratch memory.
template <int THREADS, int ITEMS, bool EXPAND, bool PAGES, typename Loader, typename Stage>
__device__ __forceinline__ void process_row(const Loader& load, int limit, int length_raw,
                                            int clamp, int topk, const ExpandMeta& m, int row,
                                            int32_t* out, TopkShared<THREADS>& sh, Stage& st,
                                            int* sel) {
  uint32_t key[ITEMS];
  int id[ITEMS];
  const RowPrefetch f =
      stage_row<THREADS, ITEMS, EXPAND, PAGES>(load, limit, m, row, key, id, sh, st);
  finish_row<THREADS, ITEMS, EXPAND, PAGES>(load, key, id, f, st, limit, length_raw, clamp, topk,
                                            m, row, out, sh, sel);
}

// Radix select and ranking of `total` compacted candidates (keys, ids and
// pages at index e of ckey / cid / cpage, in id order), C per thread.
template <int THREADS, int C, typename Emit>
__device__ __forceinline__ void select_compacted_emit(int total, int topk, uint32_t lo, uint32_t hi,
                                                      const uint32_t* ckey, const int* cid,
                                                      TopkShared<THREADS>& sh, Emit&& emit) {
  uint32_t ck[C];
  int ci[C], cp[C];
  uint32_t ccand = 0;
#pragma unroll
  for (int j = 0; j < C; ++j) {
    const int e = C * (int)threadIdx.x + j;
    const bool ok = e < total;
    ck[j] = ok ? ckey[e] : 0u;
    ci[j] = ok ? cid[e] : 0;
    cp[j] = e;
    ccand |= (uint32_t)ok << j;
  }
  radix_rank_emit<THREADS, C>(topk, lo, hi, ccand, ck, ci, cp, sh, emit);
}

template <int THREADS, int C, bool PAGES>
__device__ __forceinline__ void select_compacted(int total, int topk, uint32_t lo, uint32_t hi,
                                                 const uint32_t* ckey, const int* cid,
                                                 const int* cpage, const ExpandMeta& m,
                                                 TopkShared<THREADS>& sh, int* sel) {
  select_compacted_emit<THREADS, C>(total, topk, lo, hi, ckey, cid, sh,
                                    [&](int rank, int i, int p) {
                                      sel[rank] = i;
                                      sel[topk + rank] = PAGES ? first_slot(m, cpage[p], i) : -1;
                                    });
}

// --- expansion written by the selecting threads -----------------------------
//
// When a block's tokens map to consecutive slots from its first (logical
// token ids, or physical pages that hold whole blocks) and the causal tail's
// pages were prefetched one per thread (write_expanded's from-LDS case), the
// thread that ranks a selected block writes the block's `ratio` columns
// itself, and the columns after the selected blocks (the causal tail, then
// -1) go to the thread that prefetched the tail token's page. The row needs
// no ranked list in LDS, no barrier before it is written, and no pass over
// every column reading that list; the columns and their values are those of
// write_expanded.
__device__ __forceinline__ bool direct_expansion(const ExpandMeta& m) {
  const bool block_in_page = m.physical && (m.page_size % m.ratio == 0);
  return (!m.physical || block_in_page) && m.ratio - 1 <= kTailSlots;
}

// Columns [rank * ratio, rank * ratio + ratio) of selected block `id` (pp: the
// physical page of its first token), those below out_width; nothing for a
// rank past the span's complete blocks.
// `quads`: the row is contiguous and 16-byte aligned, ratio is a multiple of
// 4 and every complete block lies below out_width (uniform), so the block's
// columns go out as 16-byte stores.
__device__ __forceinline__ void write_block(const ExpandMeta& m, int seq, int expanded, bool quads,
                                            int rank, int id, int pp, int32_t* out) {
  const int c0 = rank * m.ratio;
  if (c0 >= expanded) return;
  const int first = id * m.ratio;
  const int s0 = m.physical ? first_slot(m, pp, id) : first;
  if (quads) {
    i32x4* dst = reinterpret_cast<i32x4*>(out + c0);
    for (int q = 0; q < m.ratio / 4; ++q) {
      i32x4 v;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int o = 4 * q + k;
        v[k] = (first + o < seq && s0 >= 0) ? s0 + o : -1;
      }
      dst[q] = v;
    }
    return;
  }
  const int n = min(m.ratio, m.out_width - c0);
  const int64_t cs = m.out_col_stride;
  for (int o = 0; o < n; ++o)
    out[(int64_t)(c0 + o) * cs] = (first + o < seq && s0 >= 0) ? s0 + o : -1;
}

// Columns [expanded, out_width): thread tid writes tail token tid with the
// page it prefetched (prefetch_tail), every other column is -1; then the
// row's count.
template <int THREADS>
__device__ __forceinline__ void write_tail(const ExpandMeta& m, const RowPrefetch& f,
                                           const ExpandedSpan& span, int row, int32_t* out) {
  static_assert(kTailSlots <= THREADS, "one tail token per thread");
  const int64_t cs = m.out_col_stride;
  const int tail = min(span.tail_count, m.ratio - 1);
  for (int c = span.expanded + (int)threadIdx.x; c < m.out_width; c += THREADS) {
    const int off = c - span.expanded;
    const int pp = m.physical ? (f.tail_ok ? f.tail_pp : -1) : 0;
    out[(int64_t)c * cs] = off < tail ? slot_of(m, f.r, span.tail_start + off, pp) : -1;
  }
  if (m.store_counts && threadIdx.x == 0) m.counts[row] = span.count(f.r);
}

// Selection of `total` compacted candidates (keys, ids and pages at index e
// of ckey / cid / cpage) with the expansion written by the selecting threads
// (direct_expansion).
template <int THREADS, int C, bool PAGES>
__device__ __forceinline__ void select_compacted_direct(int total, int topk, uint32_t lo,
                                                        uint32_t hi, const uint32_t* ckey,
                                                        const int* cid, const int* cpage,
                                                        const ExpandMeta& m, const RowPrefetch& f,
                                                        int row, int32_t* out,
                                                        TopkShared<THREADS>& sh) {
  const ExpandedSpan span = expanded_span(m, f.r, topk);
  const int seq = f.r.seq();
  const bool quads = m.out_col_stride == 1 && m.ratio % 4 == 0 && span.expanded <= m.out_width &&
                     (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  select_compacted_emit<THREADS, C>(total, topk, lo, hi, ckey, cid, sh, [&](int rank, int i, int p) {
    write_block(m, seq, span.expanded, quads, rank, i, PAGES ? cpage[p] : -1, out);
  });
  write_tail<THREADS>(m, f, span, row, out);
}

// One whole contiguous row (load.start == 0), selected without staging its
// keys. The workgroup bounds the loaded keys as select_long does (lo: the
// smallest of the full waves' floors of the m-th largest of their threads'
// maxima, at or below the k-th largest key; hi: the largest key), in the
// layout the keys were loaded in, with one barrier. Each thread then tests
// the elements it loaded (element i * THREADS + tid) against lo; the
// candidates are compacted in id order (items, then waves, then lanes)
// straight from the load layout, with their pages, after one barrier that
// exchanges the per-(item, wave) counts, and the radix select and ranking run
// on them. Against process_row this drops the staging round trip of every
// key through LDS and one barrier. Rows with too many candidates to compact
// take process_row's path with the scores already loaded.
//
// process_loaded_whole is the same row after its scores were loaded: a caller
// may issue the loads before it knows the row's length (any limit >= the
// clamped length gives the same result; elements past the length are never
// selected). `meta()` returns the row's expansion inputs and leaves the
// element pages in pg; it is called after the bound, which needs the scores
// alone, so loads it waits for can still be in flight while the bound is
// computed. DIRECT writes the expansion from the selecting threads
// (direct_expansion) when the row allows it. Returns the row's expansion
// inputs (sequence length and position).
template <int THREADS, int ITEMS, bool EXPAND, bool PAGES, bool DIRECT, typename Stage,
          typename Meta>
__device__ __forceinline__ RowMeta process_loaded_whole(const DirectLoader& load, int limit,
                                                        const uint32_t (&v)[ITEMS],
                                                        const int (&pg)[ITEMS], Meta&& meta,
                                                        int length_raw, int clamp, int topk,
                                                        const ExpandMeta& m, int row,
                                                        int32_t* out, TopkShared<THREADS>& sh,
                                                        Stage& st, int* sel) {
  constexpr int kWaves = THREADS / 64;
  constexpr int kEntries = ITEMS * kWaves;  // (item, wave) counts, item-major
  static_assert(ITEMS <= 16 && 64 % kWaves == 0, "count layout");
  // Compacted keys and ids take the key stage, their pages the page stage.
  constexpr int kCompact = ITEMS / 2 < 2 ? ITEMS / 2 : 2;
  static_assert(kCompact >= 1 && 2 * kCompact <= ITEMS, "compaction must fit the stage");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int length = length_raw > topk ? min(length_raw, clamp) : length_raw;
  constexpr uint32_t kNoBound = 0xffffffffu;
  uint32_t lo = kNoBound, hi = 0u;
  if (length > topk) {
    clear_histograms(sh);
    // Thread tid is active iff tid < length (element tid is its first); each
    // thread's maximum is one of its own elements, so a full wave's floor of
    // the m-th largest maximum is reached by m of its elements, and the full
    // waves together by m * full >= topk.
    uint32_t tmax = 0u;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
      if (i * THREADS + tid < length) tmax = max(tmax, v[i]);
    const int full = min(THREADS, length) / 64;
    const int mm = full > 0 ? (topk + full - 1) / full : 65;
    const uint32_t wf = mm <= 64 && wave < full ? wave_floor_mth_largest(tmax, mm) : kNoBound;
    const uint32_t wm = __ockl_wfred_max_u32(tid < length ? tmax : 0u);
    if (lane == 0) {
      sh.wfloor[wave] = wf;
      sh.wmax[wave] = wm;
    }
    lds_barrier();
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      lo = min(lo, sh.wfloor[w]);
      hi = max(hi, sh.wmax[w]);
    }
  }
  const RowPrefetch f = meta();
  // The expansion written by the selecting threads (uniform).
  static_assert(!DIRECT || THREADS <= 512, "the direct writer runs on all of the row's threads");
  const bool direct = DIRECT && EXPAND && (PAGES || !m.physical) && direct_expansion(m);
  if (length > topk && lo != kNoBound && lo <= hi) {
    uint32_t cand = 0;
    int below[ITEMS];  // candidates of item i in lower lanes of this wave
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const bool c = i * THREADS + tid < length && v[i] >= lo;
      cand |= (uint32_t)c << i;
      const uint64_t bal = __ballot(c);
      below[i] = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                           __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
      if (lane == 0) sh.ccount[i * kWaves + wave] = __builtin_popcountll(bal);
    }
    lds_barrier();
    // Exclusive prefix over the (item, wave) entries; entry x sits in lane
    // x % 64 of group x / 64, and item i's entries stay within group
    // i * kWaves / 64.
    constexpr int kGroups = (kEntries + 63) / 64;
    int pre[kGroups];
    int total = 0;
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
      const int x = g * 64 + lane;
      const int c = x < kEntries ? sh.ccount[x] : 0;
      const int ex = __ockl_wfscan_add_i32(c, false);
      pre[g] = total + ex;
      total += __builtin_amdgcn_readlane(ex + c, 63);
    }
    // The hints here place the rare paths (too many candidates, a row the
    // direct writer cannot take) after the common one in the code, so the
    // common path's instructions are contiguous.
    if (__builtin_expect(total <= kCompact * THREADS, 1)) {
      // Up to THREADS candidates: one per thread (the usual case, and the
      // cheapest radix passes); more: kCompact per thread.
      uint32_t* ckey = st.key;
      int* cid = reinterpret_cast<int*>(st.key + kCompact * THREADS);
      int* cpage = st.page;
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) {
        const int x = i * kWaves + wave;
        const int base = __builtin_amdgcn_readlane(pre[(i * kWaves) / 64], x % 64);
        if ((cand >> i) & 1u) {
          const int o = base + below[i];
          ckey[o] = v[i];
          cid[o] = load.start + i * THREADS + tid;
          if (PAGES) cpage[o] = pg[i];
        }
      }
      lds_barrier();
      if (__builtin_expect(direct, 1)) {
        if (__builtin_expect(kCompact == 1 || total <= THREADS, 1))
          select_compacted_direct<THREADS, 1, PAGES>(total, topk, lo, hi, ckey, cid, cpage, m, f,
                                                     row, out, sh);
        else
          select_compacted_direct<THREADS, kCompact, PAGES>(total, topk, lo, hi, ckey, cid, cpage,
                                                            m, f, row, out, sh);
        return f.r;
      }
      // A 1024-thread row hands up to 1024 candidates to its lower 512
      // threads and the upper waves end: a barrier waits only for the waves
      // that have not ended, so every radix pass, block scan and barrier of
      // the selection and the row writer spans half the waves (the
      // histogram sits at the start of the shared block in both layouts,
      // already cleared).
      if constexpr (THREADS == 1024) {
        if (total <= 1024) {
          if (__builtin_amdgcn_readfirstlane(wave) >= 8) return f.r;  // a uniform branch: the wave ends
          auto& sh2 = *reinterpret_cast<TopkShared<512>*>(&sh);
          if (total <= 512)
            select_compacted<512, 1, PAGES>(total, topk, lo, hi, ckey, cid, cpage, m, sh2, sel);
          else
            select_compacted<512, 2, PAGES>(total, topk, lo, hi, ckey, cid, cpage, m, sh2, sel);
          write_row<512, EXPAND>(f, topk, m, row, out, sh2, sel);
          return f.r;
        }
      }
      // sel shares the key stage's first 2 * topk words (topk <= total <=
      // kCompact * THREADS); radix_rank writes it after its rank scan's
      // barrier, when every candidate is in registers.
      if (kCompact == 1 || total <= THREADS)
        select_compacted<THREADS, 1, PAGES>(total, topk, lo, hi, ckey, cid, cpage, m, sh, sel);
      else
        select_compacted<THREADS, kCompact, PAGES>(total, topk, lo, hi, ckey, cid, cpage, m, sh,
                                                  sel);
      write_row<THREADS, EXPAND>(f, topk, m, row, out, sh, sel);
      return f.r;
    }
    lds_barrier();  // every wave has read the counts before they are reused
  }
  uint32_t key[ITEMS];
  int id[ITEMS];
  stage_loaded<THREADS, ITEMS, PAGES>(load, v, pg, key, id, sh, st);
  finish_row<THREADS, ITEMS, EXPAND, PAGES>(load, key, id, f, st, limit, length_raw, clamp, topk,
                                            m, row, out, sh, sel);
  return f.r;
}

// Returns the row's expansion inputs (sequence length and position).
//
// FUSED (the decode selection inside the attention's workgroups, writing the
// expanded row into LDS): the scores go out first, then the element pages
// from the guessed table row and the request (load_request), so the bound is
// computed while those are in flight, and the selecting threads write the
// expansion. Measured on decode_32k's rows it shortens the selection phase of
// each workgroup, while for rows written to global memory (the top-k kernels)
// both changes were slower: the per-block 16-byte stores to scattered
// columns cost more than the column-coalesced writer, and the later page
// loads more than the earlier bound.
template <int THREADS, int ITEMS, bool EXPAND, bool PAGES, typename Stage, bool FUSED = false>
__device__ __forceinline__ RowMeta process_row_whole(const DirectLoader& load, int limit,
                                                     int length_raw, int clamp, int topk,
                                                     const ExpandMeta& m, int row, int32_t* out,
                                                     TopkShared<THREADS>& sh, Stage& st,
                                                     int* sel) {
  uint32_t v[ITEMS];
  int pg[ITEMS];
  if constexpr (FUSED) {
    load_scores<THREADS, ITEMS>(load, limit, v);
    const RowRequest q = load_request<THREADS, ITEMS, EXPAND, PAGES>(load, limit, m, row, pg);
    return process_loaded_whole<THREADS, ITEMS, EXPAND, PAGES, true>(
        load, limit, v, pg, [&] { return load_pages<THREADS, ITEMS, EXPAND, PAGES>(load, limit, m, q, pg); },
        length_raw, clamp, topk, m, row, out, sh, st, sel);
  } else {
    const RowPrefetch f = load_row<THREADS, ITEMS, EXPAND, PAGES>(load, limit, m, row, v, pg);
    return process_loaded_whole<THREADS, ITEMS, EXPAND, PAGES, false>(
        load, limit, v, pg, [&] { return f; }, length_raw, clamp, topk, m, row, out, sh, st, sel);
  }
}

// The expansion inputs of a row (its request's sequence length, its position
// and the request's page-table row), loaded directly.
__device__ __forceinline__ RowMeta load_row_meta(const ExpandMeta& m, int row) {
  const int req = m.token_to_req[row];
  const bool mapped = req >= 0 && req < m.num_requests;
  RowMeta r;
  r.seq_len = mapped ? m.sequence_lengths[req] : 0;
  r.pos = (int)m.positions[row];
  r.table_row = m.physical ? m.table + (int64_t)(mapped ? req : 0) * m.table_row_stride : nullptr;
  return r;
}

// A row of a wide logits buffer selected by one 512-thread workgroup into an
// expanded row `out` (the decode selection inside the attention's
// workgroups, for rows longer than the 2048 keys its usual shape holds).
// As topk_adaptive_kernel with half the threads: up to 8192 keys as a whole
// row (8 or 16 keys per thread by the row's length, the selecting threads
// writing the expansion); up to 16384 staged through LDS, 32 keys per thread;
// 16385..32768 keys as exact top-k of the two halves in turn (winners kept
// in LDS), then exact top-k over the halves' winners in id order. `stage` is
// 512 x 32 keys and as many pages or winners (128 KB). Needs 2 topk <= 8192
// (the combined decode kernel allows 2 topk <= 2048).
constexpr int kWideThreads = 512;
constexpr int kWideHalf = kWideThreads * 32;
constexpr int kWideMaxColumns = 2 * kWideHalf;

__device__ __forceinline__ RowMeta select_wide_row(const float* srow, int cols, int length,
                                                   int topk, const ExpandMeta& m, int row,
                                                   int32_t* out, TopkShared<kWideThreads>& sh,
                                                   uint32_t* stage) {
  constexpr int T = kWideThreads;
  const int n = min(max(length, 0), cols);
  const int whole = max(n, 2 * topk);
  if (whole <= T * 16) {
    const DirectLoader load{srow, 0};
#define QSA_WIDE_WHOLE_ROW(ITEMS)                                                              \
  {                                                                                            \
    using Stage = TopkStage<T, ITEMS, true>;                                                   \
    auto& st = *reinterpret_cast<Stage*>(stage);                                               \
    return process_row_whole<T, ITEMS, true, true, Stage, true>(                               \
        load, n, length, cols, topk, m, row, out, sh, st, reinterpret_cast<int*>(st.key));     \
  }
    if (whole <= T * 8) QSA_WIDE_WHOLE_ROW(8)
    else QSA_WIDE_WHOLE_ROW(16)
#undef QSA_WIDE_WHOLE_ROW
  }
  if (n <= kWideHalf) {
    auto& st = *reinterpret_cast<TopkStage<T, 32, true>*>(stage);
    process_row<T, 32, true, true>(DirectLoader{srow, 0}, n, length, cols, topk, m, row, out, sh,
                                   st, reinterpret_cast<int*>(st.key));
    return load_row_meta(m, row);
  }
  // Halves [0, kWideHalf) and [kWideHalf, n); the winners (ascending ids) go
  // past the halves' key stage, the second half's after the first's, so the
  // merged list is in id order (ties go to the lower id, as in one pass).
  int* winners = reinterpret_cast<int*>(stage + T * 32);
  auto& hst = *reinterpret_cast<TopkStage<T, 32, false>*>(stage);
  int* hsel = reinterpret_cast<int*>(hst.key);
  process_row<T, 32, false, false>(DirectLoader{srow, 0}, kWideHalf, kWideHalf, kWideHalf, topk, m,
                                   row, winners, sh, hst, hsel);
  __syncthreads();
  const int rest = n - kWideHalf;
  process_row<T, 32, false, false>(DirectLoader{srow, kWideHalf}, rest, rest, rest, topk, m, row,
                                   winners + topk, sh, hst, hsel);
  __syncthreads();
  const int count = topk + min(rest, topk);
  const IndirectLoader merged{srow, winners};
  // Each thread reads its candidates' ids before it overwrites the same LDS
  // words with their pages (the page half of a 32-key stage is the winners).
  const int need = max(count, 2 * topk);
#define QSA_WIDE_MERGED(ITEMS)                                                                 \
  {                                                                                            \
    auto& st = *reinterpret_cast<TopkStage<T, ITEMS, true>*>(stage);                           \
    process_row<T, ITEMS, true, true>(merged, count, count, count, topk, m, row, out, sh, st,  \
                                      reinterpret_cast<int*>(st.key));                         \
  }
  if (need <= T * 2) QSA_WIDE_MERGED(2)
  else if (need <= T * 4) QSA_WIDE_MERGED(4)
  else if (need <= T * 8) QSA_WIDE_MERGED(8)
  else QSA_WIDE_MERGED(16)
#undef QSA_WIDE_MERGED
  return load_row_meta(m, row);
}

}  // namespace
}  // namespace qsa
