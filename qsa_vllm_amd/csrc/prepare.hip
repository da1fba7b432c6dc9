// Kernel 0: indexer preparation and cache producers, gfx950.
//
// qsa_prepare (ops/prepare.py:49-174, launch :177-225) in one launch with
// three roles, each on 16-lane row groups (lane j of a group holds dims
// 8 j .. 8 j + 7 of one 64- or 128-dim row, one 16 B load or store):
//
//  * index queries: RMSNorm + partial RoPE of every (token, index head) row
//    of the projection into a contiguous [tokens, heads, dim] output;
//  * compression groups (one per k_work item): mean of the group's raw index
//    keys (this step's projection, or the request's raw-key ring for members
//    before the chunk), RMSNorm + RoPE at the group's first position, store
//    into the compressed cache; work item 0 of a request then commits the
//    chunk's last raw keys into the ring, after its own ring reads;
//  * main K/V: copy of each (token, kv head) key and value row into its
//    cache slot.
//
// indexer_norm_rope (ops/normalization.py:33-83) is the query role alone on
// an arbitrary strided [tokens, heads, dim] input.
//
// Numerics (ops/prepare.py:16-46, ops/normalization.py:44-68). Each fp32
// product and sum rounds on its own and the post-norm steps round to bf16
// (the reference compiles with enable_fp_fusion=False), so contraction is off
// in this file. The sum of squares is formed exactly (bf16 squares are exact
// in fp32 and their sum is accumulated in double), rounded once to fp32, and
// the inverse RMS is the correctly rounded 1/sqrt: a definition the CPU
// oracle reproduces bit for bit. The reference's fp32 tree sum and
// approximate rsqrt can differ from it in the last fp32 bits, which moves a
// bf16 output by one unit only when it lies that close to a rounding
// boundary.
#pragma clang fp contract(off)

#include "qsa_common.h"
#include "../../include/qsa_hip.h"

namespace qsa {
namespace {

constexpr int kGroupLanes = 16;
constexpr int kPrepThreads = 256;
constexpr int kGroupsPerBlock = kPrepThreads / kGroupLanes;

struct NormRope {
  const uint16_t* weight;   // [dim] bf16 gamma
  const uint16_t* cos_sin;  // [max_positions, rotary] bf16: cos then sin
  int64_t max_positions;
  float eps;
  int dim;
  int rotary;
};

__device__ __forceinline__ void unpack8(const u32x4& v, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_lo(v[i]);
    f[2 * i + 1] = bf16_hi(v[i]);
  }
}

__device__ __forceinline__ u32x4 pack8(const float (&f)[8]) {
  u32x4 v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
  return v;
}

__device__ __forceinline__ float round_bf16(float x) { return bf16_lo(pack_bf16x2(x, 0.0f)); }

// Sum over the 16 lanes of a row group (lanes 16 k .. 16 k + 15).
__device__ __forceinline__ double group_sum(double v) {
#pragma unroll
  for (int m = 1; m < kGroupLanes; m <<= 1) v += __shfl_xor(v, m, kGroupLanes);
  return v;
}

// What one lane needs to normalise and rotate any row at one position: its
// gamma, cos and sin slices (raw bf16 pairs, zero outside the rotary dims or
// the table) and its rotate-half partner lane. The loads are issued here and
// consumed only when a row is rotated, so they overlap the row loads.
struct RopeLane {
  u32x4 gamma, cosr, sinr;
  int src;          // partner lane: dims d < half pair with d + half, the rest with d - half
  bool rot, first_half;
};

__device__ __forceinline__ RopeLane rope_lane(const NormRope& nr, int64_t pos, int j) {
  RopeLane r;
  const bool live = 8 * j < nr.dim;
  r.gamma = *reinterpret_cast<const u32x4*>(live ? (const void*)(nr.weight + 8 * j)
                                                 : (const void*)g_qsa_zero_rows);
  const int half = nr.rotary / 2;
  r.rot = 8 * j < nr.rotary;
  r.first_half = 8 * j < half;
  const int lane = threadIdx.x & 63;
  r.src = r.rot ? (r.first_half ? lane + half / 8 : lane - half / 8) : lane;
  const bool ok = r.rot && pos >= 0 && pos < nr.max_positions;
  const uint16_t* cs = nr.cos_sin + (ok ? pos * nr.rotary + (8 * j) % half : 0);
  r.cosr = *reinterpret_cast<const u32x4*>(ok ? (const void*)cs : (const void*)g_qsa_zero_rows);
  r.sinr = *reinterpret_cast<const u32x4*>(ok ? (const void*)(cs + half) : (const void*)g_qsa_zero_rows);
  return r;
}

// This lane's exact partial sum of squares of x (each bf16 square is exact in
// fp32, and the sums of 128 of them are exact in double).
__device__ __forceinline__ double lane_sumsq(u32x4 x) {
  float f[8];
  unpack8(x, f);
  double ss = 0.0;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss += (double)(f[i] * f[i]);
  return ss;
}

// 1 / sqrt(fp32(sum) / dim + eps), evaluated in double and rounded to fp32.
__device__ __forceinline__ float inv_rms(const NormRope& nr, double ss) {
  const float mean = __fdiv_rn((float)ss, (float)nr.dim);
  return (float)__ddiv_rn(1.0, __dsqrt_rn((double)__fadd_rn(mean, nr.eps)));
}

// RMSNorm (with the row's inverse RMS `inv`) + partial RoPE of one row held
// by a 16-lane group; lane j holds dims 8 j .. 8 j + 7 in x (zeros past the
// row). Every lane of the group must call it (it shuffles within the group).
__device__ __forceinline__ u32x4 norm_rope_scaled(const NormRope& nr, const RopeLane& rl, u32x4 x,
                                                  float inv) {
  float f[8];
  unpack8(x, f);
  float gamma[8];
  unpack8(rl.gamma, gamma);
  // Two dims per conversion: each half of a pack rounds to nearest even on
  // its own, so pairing the roundings changes no bit.
  float scaled[8];
  u32x4 sc;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t r = pack_bf16x2(f[2 * i] * inv, f[2 * i + 1] * inv);
    sc[i] = pack_bf16x2(bf16_lo(r) * gamma[2 * i], bf16_hi(r) * gamma[2 * i + 1]);
    scaled[2 * i] = bf16_lo(sc[i]);
    scaled[2 * i + 1] = bf16_hi(sc[i]);
  }
  u32x4 pr;
#pragma unroll
  for (int i = 0; i < 4; ++i) pr[i] = __builtin_amdgcn_ds_bpermute(4 * rl.src, sc[i]);
  if (!rl.rot) return sc;
  float partner[8], cosv[8], sinv[8], out[8];
  unpack8(pr, partner);
  unpack8(rl.cosr, cosv);
  unpack8(rl.sinr, sinv);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float rotated = rl.first_half ? -partner[i] : partner[i];
    const uint32_t ab = pack_bf16x2(scaled[i] * cosv[i], rotated * sinv[i]);
    out[i] = bf16_lo(ab) + bf16_hi(ab);  // rounded to bf16 by pack8
  }
  return pack8(out);
}

// The same for a row whose inverse RMS is not known yet.
__device__ __forceinline__ u32x4 norm_rope_apply(const NormRope& nr, const RopeLane& rl, u32x4 x) {
  return norm_rope_scaled(nr, rl, x, inv_rms(nr, group_sum(lane_sumsq(x))));
}

// Row load (zeros for lanes past the row or when !ok).
__device__ __forceinline__ u32x4 load_row(const uint16_t* row, int j, int dim, bool ok) {
  return *reinterpret_cast<const u32x4*>(ok && 8 * j < dim ? (const void*)(row + 8 * j)
                                                           : (const void*)g_qsa_zero_rows);
}

__device__ __forceinline__ void store_row(uint16_t* row, int j, int dim, u32x4 v) {
  if (8 * j < dim) *reinterpret_cast<u32x4*>(row + 8 * j) = v;
}

struct PrepareArgs {
  NormRope q_nr, k_nr;
  const uint16_t* index_qk;
  int64_t index_token_stride;  // elements
  int num_tokens;
  const int64_t* positions;
  int64_t position_stride;
  uint16_t* index_q_out;  // [tokens, heads, dim]
  int num_heads;
  int dim;
  // raw-key ring
  uint16_t* state;
  int64_t state_block_stride, state_token_stride;  // elements
  int state_size;
  int num_state_blocks;
  const int64_t* state_slots;
  const int32_t* state_table;
  int64_t state_table_stride;
  const int32_t* query_start_loc;
  const int64_t* logical_positions;
  int num_requests;
  // compressed keys
  uint16_t* comp;
  int64_t comp_block_stride, comp_token_stride;
  int comp_page;
  int num_comp_blocks;
  const int64_t* comp_slots;
  const int32_t* k_work;
  int num_k_work;
  int ratio;
  // main K/V
  const uint16_t* mk;
  int64_t mk_token, mk_head;
  const uint16_t* mv;
  int64_t mv_token, mv_head;
  uint16_t* mkc;
  int64_t mkc_block, mkc_token, mkc_head;
  uint16_t* mvc;
  int64_t mvc_block, mvc_token, mvc_head;
  const int64_t* main_slots;
  int main_page;
  int num_main_blocks;
  int main_heads;
  int main_dim;
  // block ranges of the roles
  int k_blocks, q_blocks;
};

// Rows a lane loads before it uses any: loads in a loop whose trip count is
// only known at run time would otherwise each wait out a round trip. The
// preparation launch loads 8 at a time: its register footprint then allows 5
// waves per SIMD instead of 3 (64 decode tokens: 8.5 against 9.2 us; the
// prefill launch the same within noise). The stand-alone compression kernel
// loads 16.
constexpr int kBatch = 8;
constexpr int kCompressBatch = 16;
// Query heads of one token per row group: they share the position's rotary
// slices, and eight rows per group keep enough bytes in flight.
constexpr int kQHeads = 8;

// Compression group `w` of request q (ops/prepare.py:120-174).
__device__ void prepare_group(const PrepareArgs& a, int q, int w, int j) {
  if (q < 0 || q >= a.num_requests) return;
  const int qs = a.query_start_loc[q];
  const int qe = a.query_start_loc[q + 1];
  const int sblock = a.state_table[(int64_t)q * a.state_table_stride];
  const int qlen = qe - qs;
  if (qlen <= 0 || qs < 0 || qe > a.num_tokens) return;
  const int64_t chunk_end = a.logical_positions[qe - 1];
  const int64_t chunk_start = chunk_end - qlen + 1;
  if (chunk_start < 0) return;
  const int R = a.ratio;
  const int64_t num_groups = (chunk_end + 1) / R - chunk_start / R;
  const int key_off = a.num_heads * a.dim;
  const bool ring_ok = sblock >= 0 && sblock < a.num_state_blocks;
  const uint16_t* ring = a.state + (int64_t)(ring_ok ? sblock : 0) * a.state_block_stride;

  if (w < num_groups) {
    const int64_t first_boundary = ((chunk_start + R) / R) * R - 1;
    const int64_t end_pos = first_boundary + (int64_t)w * R;
    const int64_t boundary_token = qs + end_pos - chunk_start;
    if (boundary_token >= qe) return;  // positions inconsistent with the chunk
    const int64_t first = end_pos - (R - 1);
    const int64_t cslot = a.comp_slots[boundary_token];
    const RopeLane rl = rope_lane(a.k_nr, first, j);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int m0 = 0; m0 < R; m0 += kBatch) {
      u32x4 v[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int64_t src_pos = first + m0 + i;
        const bool in_chunk = src_pos >= chunk_start;
        const uint16_t* row =
            in_chunk ? a.index_qk + (qs + src_pos - chunk_start) * a.index_token_stride + key_off
                     : ring + (src_pos % a.state_size) * a.state_token_stride;
        v[i] = load_row(row, j, a.dim, m0 + i < R && (in_chunk || ring_ok));
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        float f[8];
        unpack8(v[i], f);
        const bool member = m0 + i < R;
#pragma unroll
        for (int d = 0; d < 8; ++d)  // members in order, as the reference
          acc[d] = member ? acc[d] + f[d] : acc[d];
      }
    }
    float pooled[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) pooled[i] = round_bf16(__fdiv_rn(acc[i], (float)R));
    const u32x4 out = norm_rope_apply(a.k_nr, rl, pack8(pooled));
    if (cslot >= 0 && cslot / a.comp_page < a.num_comp_blocks) {
      uint16_t* dst = a.comp + (cslot / a.comp_page) * a.comp_block_stride +
                      (cslot % a.comp_page) * a.comp_token_stride;
      store_row(dst, j, a.dim, out);
    }
  }
  if (w == 0) {
    // Ring commit of the chunk's last raw keys, after this lane's ring reads
    // above (the same lane reads and writes the same dims of a ring row).
    const int suffix = min(qlen, a.state_size);
    for (int o0 = 0; o0 < suffix; o0 += kBatch) {
      u32x4 v[kBatch];
      int64_t slot[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const bool ok = o0 + i < suffix;
        const int64_t token = ok ? qe - suffix + o0 + i : qe - 1;
        const int64_t raw = a.state_slots[token];
        slot[i] = ok ? raw : -1;
        v[i] = load_row(a.index_qk + token * a.index_token_stride + key_off, j, a.dim, ok);
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        if (slot[i] >= 0 && slot[i] / a.state_size < a.num_state_blocks)
          store_row(a.state + (slot[i] / a.state_size) * a.state_block_stride +
                        (slot[i] % a.state_size) * a.state_token_stride,
                    j, a.dim, v[i]);
      }
    }
  }
}

// kQHeads query heads of one token: every row load is issued before the
// first row is normalised. The eight rows' sums of squares are reduce-scattered
// over the group (lanes 2 r and 2 r + 1 end with row r's exact sum), so one
// double-precision inverse-RMS evaluation per lane serves all eight rows, and
// row r's value is read from lane 2 r.
static_assert(kQHeads == 8 && kGroupLanes == 16, "the reduce-scatter pairs 8 rows with 16 lanes");
__device__ __forceinline__ void norm_rope_heads(const NormRope& nr, const uint16_t* token_row,
                                                int64_t head_stride, int h0, int heads,
                                                int64_t pos, bool ok, uint16_t* out_row, int j) {
  u32x4 x[kQHeads];
#pragma unroll
  for (int i = 0; i < kQHeads; ++i)
    x[i] = load_row(token_row + (int64_t)(h0 + i) * head_stride, j, nr.dim, ok && h0 + i < heads);
  const RopeLane rl = rope_lane(nr, pos, j);
  double ps[kQHeads];
#pragma unroll
  for (int i = 0; i < kQHeads; ++i) ps[i] = lane_sumsq(x[i]);
  // Each level keeps half of the rows (by one bit of j) and adds the
  // partner lane's partial sums of the same rows; the sums are exact, so the
  // order of the additions does not matter.
  const bool b3 = (j & 8) != 0, b2 = (j & 4) != 0, b1 = (j & 2) != 0;
  double s4[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const double keep = b3 ? ps[4 + t] : ps[t];
    const double give = b3 ? ps[t] : ps[4 + t];
    s4[t] = keep + __shfl_xor(give, 8, kGroupLanes);
  }
  double s2[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const double keep = b2 ? s4[2 + t] : s4[t];
    const double give = b2 ? s4[t] : s4[2 + t];
    s2[t] = keep + __shfl_xor(give, 4, kGroupLanes);
  }
  double s1 = (b1 ? s2[1] : s2[0]) + __shfl_xor(b1 ? s2[0] : s2[1], 2, kGroupLanes);
  s1 += __shfl_xor(s1, 1, kGroupLanes);  // row (j >> 1), summed over all 16 lanes
  const float inv_lane = inv_rms(nr, s1);
#pragma unroll
  for (int i = 0; i < kQHeads; ++i) {
    const float inv = __shfl(inv_lane, 2 * i, kGroupLanes);
    const u32x4 out = norm_rope_scaled(nr, rl, x[i], inv);
    if (ok && h0 + i < heads) store_row(out_row + (int64_t)(h0 + i) * nr.dim, j, nr.dim, out);
  }
}

__global__ __launch_bounds__(kPrepThreads) void prepare_kernel(const PrepareArgs a) {
  const int j = threadIdx.x & (kGroupLanes - 1);
  const int group = threadIdx.x / kGroupLanes;
  int b = blockIdx.x;
  if (b < a.k_blocks) {
    const int item = b * kGroupsPerBlock + group;
    const bool ok = item < a.num_k_work;
    const int q = ok ? a.k_work[2 * item] : -1;
    const int w = ok ? a.k_work[2 * item + 1] : 0;
    prepare_group(a, q, w, j);
    return;
  }
  b -= a.k_blocks;
  if (b < a.q_blocks) {
    const int hblocks = (a.num_heads + kQHeads - 1) / kQHeads;
    const int64_t item = (int64_t)b * kGroupsPerBlock + group;  // token * hblocks + head block
    const bool ok = item < (int64_t)a.num_tokens * hblocks;
    const int64_t token = ok ? item / hblocks : 0;
    const int h0 = ok ? (int)(item % hblocks) * kQHeads : 0;
    const int64_t pos = a.positions[token * a.position_stride];
    norm_rope_heads(a.q_nr, a.index_qk + token * a.index_token_stride, a.dim, h0, a.num_heads,
                    pos, ok, a.index_q_out + token * a.num_heads * a.dim, j);
    return;
  }
  b -= a.q_blocks;
  // Main K/V rows are already bf16 in their final coordinates (ops/prepare.py:74-95).
  const int64_t item = (int64_t)b * kGroupsPerBlock + group;  // token * heads + head
  const bool ok = item < (int64_t)a.num_tokens * a.main_heads;
  const int64_t token = ok ? item / a.main_heads : 0;
  const int head = ok ? (int)(item % a.main_heads) : 0;
  const int64_t slot = a.main_slots[token];
  const u32x4 k = load_row(a.mk + token * a.mk_token + head * a.mk_head, j, a.main_dim, ok);
  const u32x4 v = load_row(a.mv + token * a.mv_token + head * a.mv_head, j, a.main_dim, ok);
  if (!ok || slot < 0 || slot / a.main_page >= a.num_main_blocks) return;
  const int64_t blk = slot / a.main_page, off = slot % a.main_page;
  store_row(a.mkc + blk * a.mkc_block + off * a.mkc_token + head * a.mkc_head, j, a.main_dim, k);
  store_row(a.mvc + blk * a.mvc_block + off * a.mvc_token + head * a.mvc_head, j, a.main_dim, v);
}

struct NormRopeArgs {
  NormRope nr;
  const uint16_t* values;
  int64_t token_stride, head_stride;  // elements
  int tokens, heads;
  const int64_t* positions;
  int64_t position_stride;
  uint16_t* out;  // [tokens, heads, dim]
};

__global__ __launch_bounds__(kPrepThreads) void norm_rope_kernel(const NormRopeArgs a) {
  const int j = threadIdx.x & (kGroupLanes - 1);
  const int hblocks = (a.heads + kQHeads - 1) / kQHeads;
  const int64_t item = (int64_t)blockIdx.x * kGroupsPerBlock + threadIdx.x / kGroupLanes;
  const bool ok = item < (int64_t)a.tokens * hblocks;
  const int64_t token = ok ? item / hblocks : 0;
  const int h0 = ok ? (int)(item % hblocks) * kQHeads : 0;
  const int64_t pos = a.positions[token * a.position_stride];
  norm_rope_heads(a.nr, a.values + token * a.token_stride, a.head_stride, h0, a.heads, pos, ok,
                  a.out + token * a.heads * a.nr.dim, j);
}

// Rows into paged cache slots (qsa_store_cache_rows, ops/qsa.py:366-401 and
// 691-706): row r goes to slot_mapping[r] when 0 <= slot < blocks * page.
// A group copies 128 dims per step.
struct StoreRowsArgs {
  uint16_t* cache;
  int64_t block_stride, token_stride;  // elements
  int num_blocks, page, width;
  const int64_t* slots;
  const uint16_t* rows;
  int64_t row_stride;
  int num_rows;
};

__global__ __launch_bounds__(kPrepThreads) void store_rows_kernel(const StoreRowsArgs a) {
  const int j = threadIdx.x & (kGroupLanes - 1);
  const int64_t r = (int64_t)blockIdx.x * kGroupsPerBlock + threadIdx.x / kGroupLanes;
  if (r >= a.num_rows) return;
  const int64_t slot = a.slots[r];
  const bool ok = slot >= 0 && slot < (int64_t)a.num_blocks * a.page;
  const uint16_t* src = a.rows + r * a.row_stride;
  uint16_t* dst = a.cache + (ok ? (slot / a.page) * a.block_stride + (slot % a.page) * a.token_stride : 0);
  for (int c = 0; c < a.width; c += 8 * kGroupLanes) {
    const u32x4 v = load_row(src + c, j, a.width - c, ok);
    if (ok) store_row(dst + c, j, a.width - c, v);
  }
}

// Mean of the complete group ending at each row (qsa_compress_groups_with_ratio,
// ops/qsa.py:403-549 and 709-750): members from this step's rows, or from the
// request's ring before the chunk; fp32 sum in member order, divided by the
// ratio, stored as bf16 (0 for rows that close no valid group). The group's
// first position goes to 3 int64 columns: from the raw or ring position tables
// when they are given, else the position itself (0 for invalid rows).
struct CompressArgs {
  const uint16_t* raw;
  int64_t raw_row_stride;
  const int64_t* raw_pos;
  int64_t raw_pos_row_stride, raw_pos_dim_stride;
  const uint16_t* state;
  int64_t state_block_stride, state_token_stride;
  int state_size, num_state_blocks;
  const int64_t* rope;
  int64_t rope_block_stride, rope_token_stride, rope_dim_stride;
  const int32_t* state_table;
  int64_t state_table_stride;
  const int32_t* token_to_req;
  const int32_t* query_start_loc;
  int num_requests;
  const int64_t* logical_positions;
  const int64_t* compressed_slots;
  int rows, dim, ratio;
  uint16_t* pooled;
  int64_t pooled_row_stride;
  int64_t* first_positions;
  int64_t fp_row_stride, fp_col_stride;
};

__global__ __launch_bounds__(kPrepThreads) void compress_groups_kernel(const CompressArgs a) {
  const int j = threadIdx.x & (kGroupLanes - 1);
  const int row = blockIdx.x * kGroupsPerBlock + threadIdx.x / kGroupLanes;
  if (row >= a.rows) return;
  const int request = a.token_to_req[row];
  const bool req_ok = request >= 0 && request < a.num_requests;
  const int safe = req_ok ? request : 0;
  const int64_t end_pos = a.logical_positions[row];
  const int64_t cslot = a.compressed_slots[row];
  const int qs = req_ok ? a.query_start_loc[safe] : 0;
  const int qe = req_ok ? a.query_start_loc[safe + 1] : 0;
  const int sblock = req_ok ? a.state_table[(int64_t)safe * a.state_table_stride] : -1;
  const int R = a.ratio;
  const int64_t chunk_start = end_pos - (row - qs);
  const bool valid = req_ok && row >= qs && row < qe && end_pos >= R - 1 && cslot >= 0;
  const bool ring_ok = sblock >= 0 && sblock < a.num_state_blocks;
  const uint16_t* ring = a.state + (int64_t)(ring_ok ? sblock : 0) * a.state_block_stride;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int m0 = 0; m0 < R; m0 += kCompressBatch) {
    u32x4 v[kCompressBatch];
#pragma unroll
    for (int i = 0; i < kCompressBatch; ++i) {
      const int64_t position = end_pos - (R - 1) + m0 + i;
      const bool use_raw = position >= chunk_start;
      const int64_t raw_row = qs + position - chunk_start;
      const bool raw_ok = raw_row >= qs && raw_row < qe && raw_row < a.rows;
      const uint16_t* src = use_raw ? a.raw + (raw_ok ? raw_row : 0) * a.raw_row_stride
                                    : ring + (position >= 0 ? position % a.state_size : 0) *
                                                 a.state_token_stride;
      v[i] = load_row(src, j, a.dim, valid && m0 + i < R && (use_raw ? raw_ok : ring_ok));
    }
#pragma unroll
    for (int i = 0; i < kCompressBatch; ++i) {
      float f[8];
      unpack8(v[i], f);
      const bool member = m0 + i < R;
#pragma unroll
      for (int d = 0; d < 8; ++d) acc[d] = member ? acc[d] + f[d] : acc[d];
    }
  }
  float mean[8];
#pragma unroll
  for (int d = 0; d < 8; ++d) mean[d] = __fdiv_rn(acc[d], (float)R);
  store_row(a.pooled + (int64_t)row * a.pooled_row_stride, j, a.dim, pack8(mean));
  if (j < 3) {
    const int64_t first = end_pos - R + 1;
    int64_t value = valid ? first : 0;
    if (a.rope) {
      const bool from_raw = first >= chunk_start;
      const int64_t raw_first = qs + first - chunk_start;
      const bool raw_ok = valid && from_raw && raw_first >= qs && raw_first < qe && raw_first < a.rows;
      const bool ring_pos_ok = valid && !from_raw && ring_ok;
      value = raw_ok ? a.raw_pos[raw_first * a.raw_pos_row_stride + j * a.raw_pos_dim_stride]
              : ring_pos_ok ? a.rope[(int64_t)sblock * a.rope_block_stride +
                                     (first % a.state_size) * a.rope_token_stride +
                                     j * a.rope_dim_stride]
                            : 0;
    }
    a.first_positions[(int64_t)row * a.fp_row_stride + j * a.fp_col_stride] = value;
  }
}

int check_norm_rope(int dim, int rotary, int max_positions, const void* weight, const void* cos_sin,
                    const char* name) {
  if (dim != 64 && dim != 128)
    return fail(QSA_ERR_UNSUPPORTED, std::string(name) + ": index head dim must be 64 or 128");
  if (rotary < 0 || rotary > dim || rotary % 16)
    return fail(QSA_ERR_UNSUPPORTED,
                std::string(name) + ": rotary dim must be a multiple of 16 within the head dim");
  if (!weight || (rotary > 0 && (!cos_sin || max_positions <= 0)))
    return fail(QSA_ERR_INVALID, std::string(name) + ": null weight or rotary cache");
  if (((uintptr_t)weight | (uintptr_t)cos_sin) & 15u)
    return fail(QSA_ERR_INVALID, std::string(name) + ": weight and rotary cache must be 16-byte aligned");
  return QSA_OK;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace
}  // namespace qsa

using namespace qsa;

extern "C" int qsa_indexer_prepare(
    const void* index_qk, int64_t index_token_stride, int num_tokens, const int64_t* positions,
    int64_t position_stride, const void* q_norm_weight, const void* k_norm_weight,
    const void* cos_sin, int max_positions, float eps, void* index_q_out, void* state_cache,
    int64_t state_block_stride, int64_t state_token_stride, int state_size, int num_state_blocks,
    const int64_t* state_slots, const int32_t* state_table, int64_t state_table_stride,
    const int32_t* query_start_loc, const int64_t* logical_positions, int num_requests,
    void* compressed_cache, int64_t comp_block_stride, int64_t comp_token_stride,
    int comp_page_size, int num_comp_blocks, const int64_t* compressed_slots,
    const int32_t* k_work, int num_k_work, const void* main_key, int64_t main_key_token_stride,
    int64_t main_key_head_stride, const void* main_value, int64_t main_value_token_stride,
    int64_t main_value_head_stride, void* main_key_cache, int64_t main_key_cache_block_stride,
    int64_t main_key_cache_token_stride, int64_t main_key_cache_head_stride,
    void* main_value_cache, int64_t main_value_cache_block_stride,
    int64_t main_value_cache_token_stride, int64_t main_value_cache_head_stride,
    const int64_t* main_slots, int main_page_size, int num_main_blocks, int num_index_heads,
    int index_head_dim, int rotary_dim, int compress_ratio, int main_kv_heads,
    int main_head_dim, void* stream) {
  const char* name = "qsa_indexer_prepare";
  if (num_tokens < 0 || num_k_work < 0) return fail(QSA_ERR_INVALID, "qsa_indexer_prepare: negative size");
  if (num_tokens == 0 && num_k_work == 0) return QSA_OK;
  int st = check_norm_rope(index_head_dim, rotary_dim, max_positions, q_norm_weight, cos_sin, name);
  if (st != QSA_OK) return st;
  if (!k_norm_weight || !aligned16(k_norm_weight))
    return fail(QSA_ERR_INVALID, "qsa_indexer_prepare: k_norm_weight must be a 16-byte aligned pointer");
  if (num_index_heads <= 0 || compress_ratio <= 0 || state_size <= 0 || comp_page_size <= 0 ||
      main_page_size <= 0 || main_kv_heads < 0)
    return fail(QSA_ERR_INVALID, "qsa_indexer_prepare: bad head count, ratio or page size");
  if (main_kv_heads > 0 && main_head_dim != 64 && main_head_dim != 128)
    return fail(QSA_ERR_UNSUPPORTED, "qsa_indexer_prepare: main head dim must be 64 or 128");
  if (!index_qk || !positions || !index_q_out ||
      (num_k_work > 0 && (!state_cache || !state_slots || !state_table || !query_start_loc ||
                          !logical_positions || !compressed_cache || !compressed_slots || !k_work)) ||
      (main_kv_heads > 0 && num_tokens > 0 &&
       (!main_key || !main_value || !main_key_cache || !main_value_cache || !main_slots)))
    return fail(QSA_ERR_INVALID, "qsa_indexer_prepare: null tensor pointer");
  if (!aligned16(index_qk) || !aligned16(index_q_out) || !aligned16(state_cache) ||
      !aligned16(compressed_cache) || !aligned16(main_key) || !aligned16(main_value) ||
      !aligned16(main_key_cache) || !aligned16(main_value_cache) ||
      (index_token_stride | state_block_stride | state_token_stride | comp_block_stride |
       comp_token_stride | main_key_token_stride | main_key_head_stride | main_value_token_stride |
       main_value_head_stride | main_key_cache_block_stride | main_key_cache_token_stride |
       main_key_cache_head_stride | main_value_cache_block_stride |
       main_value_cache_token_stride | main_value_cache_head_stride) & 7)
    return fail(QSA_ERR_INVALID,
                "qsa_indexer_prepare: tensors must be 16-byte aligned with strides that are "
                "multiples of 8 elements and unit dim stride");
  PrepareArgs a = {};
  a.q_nr = NormRope{static_cast<const uint16_t*>(q_norm_weight),
                    static_cast<const uint16_t*>(cos_sin), max_positions, eps, index_head_dim,
                    rotary_dim};
  a.k_nr = a.q_nr;
  a.k_nr.weight = static_cast<const uint16_t*>(k_norm_weight);
  a.index_qk = static_cast<const uint16_t*>(index_qk);
  a.index_token_stride = index_token_stride;
  a.num_tokens = num_tokens;
  a.positions = positions;
  a.position_stride = position_stride;
  a.index_q_out = static_cast<uint16_t*>(index_q_out);
  a.num_heads = num_index_heads;
  a.dim = index_head_dim;
  a.state = static_cast<uint16_t*>(state_cache);
  a.state_block_stride = state_block_stride;
  a.state_token_stride = state_token_stride;
  a.state_size = state_size;
  a.num_state_blocks = num_state_blocks;
  a.state_slots = state_slots;
  a.state_table = state_table;
  a.state_table_stride = state_table_stride;
  a.query_start_loc = query_start_loc;
  a.logical_positions = logical_positions;
  a.num_requests = num_requests;
  a.comp = static_cast<uint16_t*>(compressed_cache);
  a.comp_block_stride = comp_block_stride;
  a.comp_token_stride = comp_token_stride;
  a.comp_page = comp_page_size;
  a.num_comp_blocks = num_comp_blocks;
  a.comp_slots = compressed_slots;
  a.k_work = k_work;
  a.num_k_work = num_k_work;
  a.ratio = compress_ratio;
  a.mk = static_cast<const uint16_t*>(main_key);
  a.mk_token = main_key_token_stride;
  a.mk_head = main_key_head_stride;
  a.mv = static_cast<const uint16_t*>(main_value);
  a.mv_token = main_value_token_stride;
  a.mv_head = main_value_head_stride;
  a.mkc = static_cast<uint16_t*>(main_key_cache);
  a.mkc_block = main_key_cache_block_stride;
  a.mkc_token = main_key_cache_token_stride;
  a.mkc_head = main_key_cache_head_stride;
  a.mvc = static_cast<uint16_t*>(main_value_cache);
  a.mvc_block = main_value_cache_block_stride;
  a.mvc_token = main_value_cache_token_stride;
  a.mvc_head = main_value_cache_head_stride;
  a.main_slots = main_slots;
  a.main_page = main_page_size;
  a.num_main_blocks = num_main_blocks;
  a.main_heads = main_kv_heads;
  a.main_dim = main_head_dim;
  const int64_t k_blocks = ((int64_t)num_k_work + kGroupsPerBlock - 1) / kGroupsPerBlock;
  const int64_t q_items = (int64_t)num_tokens * ((num_index_heads + kQHeads - 1) / kQHeads);
  const int64_t q_blocks = (q_items + kGroupsPerBlock - 1) / kGroupsPerBlock;
  const int64_t m_blocks = ((int64_t)num_tokens * main_kv_heads + kGroupsPerBlock - 1) / kGroupsPerBlock;
  const int64_t blocks = k_blocks + q_blocks + m_blocks;
  if (blocks > INT32_MAX) return fail(QSA_ERR_UNSUPPORTED, "qsa_indexer_prepare: grid too large");
  if (num_tokens == 0 && num_k_work > 0)
    return fail(QSA_ERR_INVALID, "qsa_indexer_prepare: compression work without tokens");
  a.k_blocks = (int)k_blocks;
  a.q_blocks = (int)q_blocks;
  hipLaunchKernelGGL(prepare_kernel, dim3((unsigned)blocks), dim3(kPrepThreads), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("qsa_indexer_prepare launch");
}

extern "C" int qsa_indexer_norm_rope(const void* values, int64_t token_stride, int64_t head_stride,
                                     int tokens, int heads, int dim, const void* weight,
                                     const int64_t* positions, int64_t position_stride,
                                     const void* cos_sin, int max_positions, float eps,
                                     int rotary_dim, void* out, void* stream) {
  const char* name = "qsa_indexer_norm_rope";
  if (tokens < 0 || heads < 0) return fail(QSA_ERR_INVALID, "qsa_indexer_norm_rope: negative size");
  if (tokens == 0 || heads == 0) return QSA_OK;
  int st = check_norm_rope(dim, rotary_dim, max_positions, weight, cos_sin, name);
  if (st != QSA_OK) return st;
  if (!values || !positions || !out) return fail(QSA_ERR_INVALID, "qsa_indexer_norm_rope: null tensor pointer");
  if (!aligned16(values) || !aligned16(out) || ((token_stride | head_stride) & 7))
    return fail(QSA_ERR_INVALID,
                "qsa_indexer_norm_rope: values and out must be 16-byte aligned with strides that "
                "are multiples of 8 elements and unit dim stride");
  const int64_t items = (int64_t)tokens * ((heads + kQHeads - 1) / kQHeads);
  const int64_t blocks = (items + kGroupsPerBlock - 1) / kGroupsPerBlock;
  if (blocks > INT32_MAX) return fail(QSA_ERR_UNSUPPORTED, "qsa_indexer_norm_rope: grid too large");
  NormRopeArgs a;
  a.nr = NormRope{static_cast<const uint16_t*>(weight), static_cast<const uint16_t*>(cos_sin),
                  max_positions, eps, dim, rotary_dim};
  a.values = static_cast<const uint16_t*>(values);
  a.token_stride = token_stride;
  a.head_stride = head_stride;
  a.tokens = tokens;
  a.heads = heads;
  a.positions = positions;
  a.position_stride = position_stride;
  a.out = static_cast<uint16_t*>(out);
  hipLaunchKernelGGL(norm_rope_kernel, dim3((unsigned)blocks), dim3(kPrepThreads), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("qsa_indexer_norm_rope launch");
}

extern "C" int qsa_store_cache_rows(void* cache, int64_t cache_block_stride,
                                    int64_t cache_token_stride, int num_blocks, int page_size,
                                    int width, const int64_t* slot_mapping, const void* rows,
                                    int64_t row_stride, int num_rows, void* stream) {
  if (num_rows < 0) return fail(QSA_ERR_INVALID, "qsa_store_cache_rows: negative rows");
  if (num_rows == 0) return QSA_OK;
  if (!cache || !slot_mapping || !rows) return fail(QSA_ERR_INVALID, "qsa_store_cache_rows: null tensor pointer");
  if (page_size <= 0 || num_blocks < 0 || width <= 0 || width % 8)
    return fail(QSA_ERR_UNSUPPORTED, "qsa_store_cache_rows: width must be a positive multiple of 8");
  if (!aligned16(cache) || !aligned16(rows) || ((cache_block_stride | cache_token_stride | row_stride) & 7))
    return fail(QSA_ERR_INVALID,
                "qsa_store_cache_rows: cache and rows must be 16-byte aligned with strides that "
                "are multiples of 8 elements and unit dim stride");
  StoreRowsArgs a{static_cast<uint16_t*>(cache), cache_block_stride, cache_token_stride, num_blocks,
                  page_size, width, slot_mapping, static_cast<const uint16_t*>(rows), row_stride,
                  num_rows};
  hipLaunchKernelGGL(store_rows_kernel, dim3((num_rows + kGroupsPerBlock - 1) / kGroupsPerBlock),
                     dim3(kPrepThreads), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("qsa_store_cache_rows launch");
}

extern "C" int qsa_compress_groups(
    const void* raw_keys, int64_t raw_row_stride, const int64_t* raw_positions,
    int64_t raw_pos_row_stride, int64_t raw_pos_dim_stride, const void* state_cache,
    int64_t state_block_stride, int64_t state_token_stride, int state_size, int num_state_blocks,
    const int64_t* rope_positions, int64_t rope_block_stride, int64_t rope_token_stride,
    int64_t rope_dim_stride, const int32_t* state_table, int64_t state_table_stride,
    const int32_t* token_to_req, const int32_t* query_start_loc, int num_requests,
    const int64_t* logical_positions, const int64_t* compressed_slots, int rows, int head_dim,
    int compress_ratio, void* pooled, int64_t pooled_row_stride, int64_t* first_positions,
    int64_t first_positions_row_stride, int64_t first_positions_col_stride, void* stream) {
  if (rows < 0) return fail(QSA_ERR_INVALID, "qsa_compress_groups: negative rows");
  if (rows == 0) return QSA_OK;
  if (head_dim != 64 && head_dim != 128)
    return fail(QSA_ERR_UNSUPPORTED, "qsa_compress_groups: head dim must be 64 or 128");
  if (compress_ratio <= 0 || state_size <= 0)
    return fail(QSA_ERR_INVALID, "qsa_compress_groups: ratio and ring size must be positive");
  if (!raw_keys || !state_cache || !state_table || !token_to_req || !query_start_loc ||
      !logical_positions || !compressed_slots || !pooled || !first_positions ||
      (rope_positions && !raw_positions))
    return fail(QSA_ERR_INVALID, "qsa_compress_groups: null tensor pointer");
  if (!aligned16(raw_keys) || !aligned16(state_cache) || !aligned16(pooled) ||
      ((raw_row_stride | state_block_stride | state_token_stride | pooled_row_stride) & 7))
    return fail(QSA_ERR_INVALID,
                "qsa_compress_groups: keys, ring and output must be 16-byte aligned with strides "
                "that are multiples of 8 elements and unit dim stride");
  CompressArgs a{static_cast<const uint16_t*>(raw_keys), raw_row_stride, raw_positions,
                 raw_pos_row_stride, raw_pos_dim_stride, static_cast<const uint16_t*>(state_cache),
                 state_block_stride, state_token_stride, state_size, num_state_blocks,
                 rope_positions, rope_block_stride, rope_token_stride, rope_dim_stride,
                 state_table, state_table_stride, token_to_req, query_start_loc, num_requests,
                 logical_positions, compressed_slots, rows, head_dim, compress_ratio,
                 static_cast<uint16_t*>(pooled), pooled_row_stride, first_positions,
                 first_positions_row_stride, first_positions_col_stride};
  hipLaunchKernelGGL(compress_groups_kernel, dim3((rows + kGroupsPerBlock - 1) / kGroupsPerBlock),
                     dim3(kPrepThreads), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("qsa_compress_groups launch");
}
