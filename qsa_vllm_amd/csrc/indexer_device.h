// Device side of the QSA indexer score.
//
// logits[r, c] = D^-0.5 * sum_h relu(q[r, h, :] . K[c, :]) over the visible
// compressed keys of row r (ops/indexer.py:24-114 decode, :117-223 prefill),
// bf16 inputs, fp32 accumulation.
//
// v_mfma_f32_32x32x16_bf16 with the index heads on M and 32 keys on N:
// A = Q[32 heads][16 dims] stays in registers for the whole row, B = K^T[16
// dims][32 keys] is one 16 B load per lane per K step. The 32x32 accumulator
// holds 16 heads of one key per lane, so the ReLU head-sum is 16 in-lane adds
// plus one cross-half shuffle, and lanes 0..31 then hold the 32 logits of the
// tile.
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

__device__ __forceinline__ float relu_head_sum(const f32x16& acc) {
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += fmaxf(acc[i], 0.0f);
  return s;
}

// A operand: lane holds Q[row][head 32 mb + kk][16 s + 8 half .. +7]; heads
// past num_heads read the zero block.
template <int D, int MB>
__device__ __forceinline__ void load_q(const IndexerParams& p, int row, bf16x8 (&qa)[MB][D / 16]) {
  const int kk = threadIdx.x & 31;
  const int half = (threadIdx.x >> 5) & 1;
  const char* zero = reinterpret_cast<const char*>(g_qsa_zero_rows);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int h = 32 * mb + kk;
    const uint16_t* qrow = p.q + (int64_t)row * p.q_row + (int64_t)h * p.q_head;
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
      const void* src = h < p.num_heads ? (const void*)(qrow + 16 * s + 8 * half) : (const void*)zero;
      qa[mb][s] = __builtin_bit_cast(bf16x8, load_u32x4(src));
    }
  }
}

// Issues the loads of one 32-key tile's B operand: this lane's key c (page
// entry `page` of its request, live when c is visible), 16 B per K step.
template <int D>
__device__ __forceinline__ void issue_key_tile(const IndexerParams& p, int c, int page, bool live,
                                               bf16x8 (&kb)[D / 16]) {
  const int half = (threadIdx.x >> 5) & 1;
  const int lp = p.page_div.div(c);
  const bool ok = live && page >= 0 && page < p.num_blocks;
  const char* kp = ok ? p.k + (int64_t)page * p.kb + (int64_t)(c - lp * p.cache_page) * p.kt
                      : reinterpret_cast<const char*>(g_qsa_zero_rows);
#pragma unroll
  for (int s = 0; s < D / 16; ++s)
    kb[s] = __builtin_bit_cast(bf16x8, load_u32x4(kp + (16 * s + 8 * half) * 2));
}

// Page-table entry of this lane's key c (zero block when c is not visible).
__device__ __forceinline__ int key_page(const IndexerParams& p, const int32_t* trow, int c,
                                        bool live) {
  return *(live ? trow + p.page_div.div(c) : reinterpret_cast<const int32_t*>(g_qsa_zero_rows));
}

// The logit of this lane's key (valid in lanes 0..31): ReLU head-sum of the
// 32x32 tile product, one cross-half shuffle, times D^-0.5.
template <int D, int MB>
__device__ __forceinline__ float tile_logit(const IndexerParams& p, const bf16x8 (&qa)[MB][D / 16],
                                            const bf16x8 (&kb)[D / 16]) {
  float sum = 0.0f;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    f32x16 acc = {};
#pragma unroll
    for (int s = 0; s < D / 16; ++s)
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa[mb][s], kb[s], acc, 0, 0, 0);
    sum += relu_head_sum(acc);
  }
  sum += shfl_xor_f(sum, 32);
  return sum * p.scale;
}

// Scores TPW consecutive 32-key tiles of one row starting at tile0 (keys
// c < vis are live; trow is the row's page-table row) and calls
// sink(c, logit) for every live key, from lanes 0..31.
//
// A wave's loads complete in issue order, so they are issued in the order
// they are needed and all before the first use: the page-table entries of
// the wave's keys, then every key row. Each wait then covers exactly the
// group in hand while the rest stays in flight. All loads are unconditional
// (invalid keys read the zero block), which keeps the wait counts static.
template <int D, int MB, int TPW, typename Sink>
__device__ __forceinline__ void score_tiles(const IndexerParams& p, const int32_t* trow, int tile0,
                                            int vis, const bf16x8 (&qa)[MB][D / 16], Sink sink) {
  const int kk = threadIdx.x & 31;
  const int half = (threadIdx.x >> 5) & 1;
  int page[TPW];
  bool live[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int c = (tile0 + t) * 32 + kk;
    live[t] = c < vis;
    page[t] = key_page(p, trow, c, live[t]);
  }
  bf16x8 kb[TPW][D / 16];
#pragma unroll
  for (int t = 0; t < TPW; ++t) issue_key_tile<D>(p, (tile0 + t) * 32 + kk, page[t], live[t], kb[t]);
  __builtin_amdgcn_sched_barrier(0);  // keep every load ahead of the first MFMA
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const float v = tile_logit<D, MB>(p, qa, kb[t]);
    const int c = (tile0 + t) * 32 + kk;
    if (half == 0 && live[t]) sink(c, v);
  }
}

}  // namespace
}  // namespace qsa
