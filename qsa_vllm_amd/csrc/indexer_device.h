// Device side of the QSA indexer score.
//
// logits[r, c] = D^-0.5 * sum_h relu(q[r, h, :] . K[c, :]) over the visible
// compressed keys of row r (ops/indexer.py:24-114 decode, :117-223 prefill),
// bf16 inputs, fp32 accumulation.
//
#pragma once

#include "qsa_common.h"

namespace qsa {
namespace {

struct IndexerParams {
  const uint16_t* q;
  int64_t q_row, q_head;  // elements
  const char* k;
  int64_t kb, kt;  // bytes
  int num_blocks;
  int cache_page;
  FastDiv page_div;
  const int32_t* table;
  int64_t table_row;
  int table_width;
  const int32_t* visible;
  int num_heads;
  int decode_query_len;
  float* logits;
  int64_t logits_row;
  int logits_cols;
  float scale;
  // prefill only
  const int32_t* query_start_loc;
  int num_requests;
  int query_offset;
  int num_rows;
  int key_tiles_per_wg;
};

// Byte address of compressed key c of a request, or the zero block.
__device__ __forceinline__ const char* key_ptr(const IndexerParams& p, const int32_t* trow, int c,
                                               bool live) {
  const char* zero = reinterpret_cast<const char*>(g_qsa_zero_rows);
  if (!live) return zero;
  const int lp = p.page_div.div(c);
  const int off = c - lp * p.cache_page;
  const int page = trow[lp];
  if (page < 0 || page >= p.num_blocks) return zero;
  return p.k + (int64_t)page * p.kb + (int64_t)off * p.kt;
}

// max(x, 0) as a signed-integer max of the fp32 bits: equal to the float
// ReLU for every non-NaN x (negative floats, -0.0 included, are negative
// integers) in one v_max_i32, where fmaxf first quiets its operand (a second
// VALU op under IEEE mode).
__device__ __forceinline__ float relu_f32(float x) {
  return __int_as_float(max(__float_as_int(x), 0));
}

// Sum of the ReLU of a lane's 16 accumulator heads, as a pairwise tree (four
// dependent adds instead of sixteen).
__device__ __forceinline__ float relu_head_sum(const f32x16& acc) {
  float r[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) r[i] = relu_f32(acc[i]);
#pragma unroll
  for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
    for (int i = 0; i < w; ++i) r[i] += r[i + w];
  return r[0];
}

// ---------------------------------------------------------------------------
// Decode scoring: v_mfma_f32_16x16x32_bf16 with 16 index heads on M and 16
// keys on N. B = K^T[32 dims][16 keys]: lane (n, g) = (lane & 15, lane >> 4)
// holds key n's dims 32 s + 8 g .. +7, so one load instruction reads 16 keys
// x 64 contiguous bytes (a wave streams whole 256 B key rows in 4 loads). A =
// Q[16 heads][32 dims] per head block stays in registers. The 16x16
// accumulator gives lane (n, g) heads 4 g .. 4 g + 3 of key n: the ReLU
// head-sum is in-lane adds over head blocks and those 4 heads plus two
// cross-group shuffles, after which lanes 0..15 hold 16 consecutive logits.
// ---------------------------------------------------------------------------
constexpr int kKeysPerTile = 16;

// A operand for head block hb: lane (m, g) holds Q[row][16 hb + m][32 s + 8 g
// .. +7]; heads past num_heads read the zero block.
template <int D, int HB>
__device__ __forceinline__ void load_q(const IndexerParams& p, int row, bf16x8 (&qa)[HB][D / 32]) {
  const int m = threadIdx.x & 15;
  const int g = (threadIdx.x >> 4) & 3;
  const char* zero = reinterpret_cast<const char*>(g_qsa_zero_rows);
#pragma unroll
  for (int hb = 0; hb < HB; ++hb) {
    const int h = 16 * hb + m;
    const uint16_t* qrow = p.q + (int64_t)row * p.q_row + (int64_t)h * p.q_head;
#pragma unroll
    for (int s = 0; s < D / 32; ++s) {
      const void* src = h < p.num_heads ? (const void*)(qrow + 32 * s + 8 * g) : (const void*)zero;
      qa[hb][s] = __builtin_bit_cast(bf16x8, load_u32x4(src));
    }
  }
}

// Page-table entry of key c (zero block when c is not visible).
__device__ __forceinline__ int key_page(const IndexerParams& p, const int32_t* trow, int c,
                                        bool live) {
  return *(live ? trow + p.page_div.div(c) : reinterpret_cast<const int32_t*>(g_qsa_zero_rows));
}

// Issues the B-operand loads of this lane's key c of a tile.
template <int D>
__device__ __forceinline__ void issue_key_tile(const IndexerParams& p, int c, int page, bool live,
                                               bf16x8 (&kb)[D / 32]) {
  const int g = (threadIdx.x >> 4) & 3;
  const int lp = p.page_div.div(c);
  const bool ok = live && page >= 0 && page < p.num_blocks;
  const char* kp = ok ? p.k + (int64_t)page * p.kb + (int64_t)(c - lp * p.cache_page) * p.kt
                      : reinterpret_cast<const char*>(g_qsa_zero_rows);
#pragma unroll
  for (int s = 0; s < D / 32; ++s)
    kb[s] = __builtin_bit_cast(bf16x8, load_u32x4(kp + (32 * s + 8 * g) * 2));
}

// The logit of this lane's key (every lane of a 16-lane column holds it).
template <int D, int HB>
__device__ __forceinline__ float tile_logit(const IndexerParams& p, const bf16x8 (&qa)[HB][D / 32],
                                            const bf16x8 (&kb)[D / 32]) {
  float sum = 0.0f;
#pragma unroll
  for (int hb = 0; hb < HB; ++hb) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < D / 32; ++s)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[hb][s], kb[s], acc, 0, 0, 0);
    sum += (relu_f32(acc[0]) + relu_f32(acc[1])) + (relu_f32(acc[2]) + relu_f32(acc[3]));
  }
  sum += shfl_xor_f(sum, 16);
  return sum_wave_halves(sum) * p.scale;
}

// Scores TPW consecutive 16-key tiles of one row starting at tile0 (keys
// c < vis are live; trow is the row's page-table row) and calls
// sink(c, logit) for every live key, from lanes 0..15.
//
// A wave's loads complete in issue order, so they are issued in the order
// they are needed and all before the first use: the page-table entries of
// the wave's keys, then every key row. Each wait then covers exactly the
// group in hand while the rest stays in flight. All loads are unconditional
// (invalid keys read the zero block), which keeps the wait counts static.
template <int D, int HB, int TPW, typename Sink>
__device__ __forceinline__ void score_tiles(const IndexerParams& p, const int32_t* trow, int tile0,
                                            int vis, const bf16x8 (&qa)[HB][D / 32], Sink sink) {
  const int n = threadIdx.x & 15;
  int page[TPW];
  bool live[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int c = (tile0 + t) * kKeysPerTile + n;
    live[t] = c < vis;
    page[t] = key_page(p, trow, c, live[t]);
  }
  bf16x8 kb[TPW][D / 32];
#pragma unroll
  for (int t = 0; t < TPW; ++t)
    issue_key_tile<D>(p, (tile0 + t) * kKeysPerTile + n, page[t], live[t], kb[t]);
  __builtin_amdgcn_sched_barrier(0);  // keep every load ahead of the first MFMA
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const float v = tile_logit<D, HB>(p, qa, kb[t]);
    const int c = (tile0 + t) * kKeysPerTile + n;
    if (threadIdx.x < 16 && live[t]) sink(c, v);
  }
}

// s_waitcnt immediate that waits for the vector-memory counter alone (gfx9
// encoding: vmcnt in bits 3:0 and 15:14, expcnt and lgkmcnt at their maxima).
constexpr int ix_vmcnt_only(int n) { return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14); }

// Waits until at most n (a multiple of 4 below 32, constant once the caller's
// loop is unrolled) vector-memory operations are in flight.
__device__ __forceinline__ void wait_vmcnt_quads(int n) {
  switch (n) {
    case 0: __builtin_amdgcn_s_waitcnt(ix_vmcnt_only(0)); break;
    case 4: __builtin_amdgcn_s_waitcnt(ix_vmcnt_only(4)); break;
    case 8: __builtin_amdgcn_s_waitcnt(ix_vmcnt_only(8)); break;
    case 12: __builtin_amdgcn_s_waitcnt(ix_vmcnt_only(12)); break;
    case 16: __builtin_amdgcn_s_waitcnt(ix_vmcnt_only(16)); break;
    case 20: __builtin_amdgcn_s_waitcnt(ix_vmcnt_only(20)); break;
    case 24: __builtin_amdgcn_s_waitcnt(ix_vmcnt_only(24)); break;
    default: __builtin_amdgcn_s_waitcnt(ix_vmcnt_only(28)); break;
  }
}

// score_tiles with the keys moved straight into LDS (D = 128, a cache page of
// a multiple of 16 keys, so a tile's keys share one page-table entry).
// global_load_lds_dwordx4 writes lane l's 16 bytes at the destination + 16 l,
// so instruction i of a tile moves keys 4 i .. 4 i + 3 as whole 256 B rows
// (lane (n, g) loads unit n ^ (4 i + g) of key 4 i + g): four full rows per
// instruction instead of the B operand's 16 keys x 64 bytes, which a CU's
// texture path streams at about half the rate. Unit c of key m then sits at
// position c ^ m of its row, so the B-operand reads (lane (n, g): unit 4 s +
// g of key n) are conflict-free. The data never passes through VGPRs; each
// tile's reads wait (vmcnt) only for that tile's four loads. `region`: the
// wave's TPW x 4 KB of LDS.
template <int HB, int TPW, typename Sink>
__device__ __forceinline__ void score_tiles_dma(const IndexerParams& p, const int32_t* trow,
                                                int tile0, int vis, const bf16x8 (&qa)[HB][4],
                                                char* region, Sink sink) {
  static_assert(TPW <= 8, "at most 28 loads behind a tile");
  constexpr int kTileBytes = kKeysPerTile * 256;
  const int n = threadIdx.x & 15;
  const int g = (threadIdx.x >> 4) & 3;
  const char* zero = reinterpret_cast<const char*>(g_qsa_zero_rows);
  const int32_t* zero_i = reinterpret_cast<const int32_t*>(g_qsa_zero_rows);
  // Every read of the region from a previous call has completed before the
  // new rows overwrite it.
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  __builtin_amdgcn_sched_barrier(0);
  // Lane t < TPW loads tile t's page-table entry (one load, one wait); the
  // tiles' pages are then read from those lanes.
  const int tl = (int)(threadIdx.x % TPW);
  const int cl = (tile0 + tl) * kKeysPerTile;
  const int page_l = *(cl < vis ? trow + p.page_div.div(cl) : zero_i);
  int page[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) page[t] = __builtin_amdgcn_readlane(page_l, t);
  // This lane's byte offsets within a tile's first key, the same for every
  // tile: instruction i, key 4 i + g, unit n ^ key.
  int64_t loff[4];
  int zoff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int key = 4 * i + g;
    zoff[i] = 16 * (n ^ key);
    loff[i] = (int64_t)key * p.kt + zoff[i];
  }
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int c0 = (tile0 + t) * kKeysPerTile;
    const int off0 = c0 - p.page_div.div(c0) * p.cache_page;
    const bool page_ok = page[t] >= 0 && page[t] < p.num_blocks;
    const char* base = p.k + (int64_t)page[t] * p.kb + (int64_t)off0 * p.kt;  // uniform
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool ok = page_ok && c0 + 4 * i + g < vis;
      const char* src = ok ? base + loff[i] : zero + zoff[i];
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void*)src,
          (__attribute__((address_space(3))) void*)(region + t * kTileBytes + i * 1024), 16, 0,
          0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // The logits are stored after the last tile: a store counts as a vector
  // memory operation too, and one issued between the tiles would make each
  // later tile's wait cover it as well.
  float val[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    // Tile t has landed once at most the later tiles' loads are in flight.
    wait_vmcnt_quads(4 * (TPW - 1 - t));
    __builtin_amdgcn_sched_barrier(0);
    bf16x8 kb[4];
    const char* krow = region + t * kTileBytes + n * 256;
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2)
      kb[s2] = __builtin_bit_cast(
          bf16x8, *reinterpret_cast<const u32x4*>(krow + 16 * ((4 * s2 + g) ^ n)));
    val[t] = tile_logit<128, HB>(p, qa, kb);
  }
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int c = (tile0 + t) * kKeysPerTile + n;
    if (threadIdx.x < 16 && c < vis) sink(c, val[t]);
  }
}

}  // namespace
}  // namespace qsa
