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

}  // namespace
}  // namespace qsa
