// Kernel 3: bf16 paged sparse GQA attention over selected KV slots, gfx950.
//
// Behaviour follows ops/qsa.py:109-362 and :594-688 of the reference plugin
// (split-K online softmax in the log2 domain, P rounded to bf16 before P.V,
// normalised fp32 partials + log2-LSE merge, optional bf16(o)*sigmoid(gate)).
//
// Work decomposition. One workgroup of WAVES waves handles (row, split, head
// group). A head group is 16 query-head slots sharing NKV kv heads (GQA group
// G, NKV*G <= 16). Each wave walks 32-token tiles of the row's index list:
//
//   S^T[tok][head] = K_tile (A, 16 tokens x 32 dims) * Q^T (B, 32 dims x 16 heads)
//       v_mfma_f32_16x16x32_bf16; K rows are loaded whole, like V's, into the
//       wave's LDS region (straight into LDS for logical rows with D = 128,
//       through registers for physical rows) and read back in the A layout
//       (D = 64 logical rows load the A layout straight from memory, 64 B
//       contiguous per token per instruction); one accumulator per kv head,
//       each lane keeping the one its head attends with.
//   O^T[dim][head] += V_tile^T (A, 16 dims x 32 tokens) * P^T (B, 32 tok x 16 heads)
//       each lane loads an 8 token x DPL dim block of V (one 16 B row load per
//       token) and transposes it in registers with v_perm_b32; P^T is exactly
//       the lane's own softmax numerators, so P never leaves registers and the
//       per-head rescale factor lives in the lane that owns that head.
//
// Index entries. A lane loads the index entries of its two K tokens only; the
// slots of its eight V tokens are K slots of lanes in the same 16-lane row
// and arrive by ds_bpermute.
//
// Load schedule. A wave's global loads complete in issue order, so the tile
// loop is a two-stage pipeline over the K and V halves of a tile:
//
//   Q.K + softmax (t) | slots, issue K (t+W) | P.V (t) |
//   issue index loads (t+2W), permute V slots, issue V (t+W)
//
// Logical indices add a third stage for their block-table entries (index
// entries of t+3W, table entries of t+2W, K/V of t+W in flight), so the table
// loads never wait behind the tile in flight.
//
// Every wait is for the oldest group in flight, and the next tile's K (V)
// bytes stream in while P.V (the next Q.K) computes, so a wave never leaves
// the memory system idle behind its own arithmetic. sched_barrier pins that
// issue order against the scheduler. Invalid slots read a block of zeros in
// device memory instead of K/V, so no per-element masking is needed beyond
// the -inf score.
//
// The waves merge (max, sum, O) through LDS. With one split the workgroup
// writes the bf16 output (and gate); with several it writes an fp32 partial +
// log2-LSE and a second kernel merges them. Merging in the last-arriving
// workgroup instead was measured slower on gfx950: device-scope release
// fences write back the XCD's L2, and write-through partial stores cost more
// than the second launch.
#include "qsa_common.h"
#include "topk_device.h"
#include "../../include/qsa_hip.h"

#include <algorithm>
#include <cstring>
#include <mutex>

// The combined decode kernel for wide logits buffers lives in its own code
// object (sparse_attn_wide.hip compiles this file with QSA_ATTN_WIDE_UNIT):
// its long-row selection is over a megabyte of code, and with it in this
// file's code object the 2048-column kernel - the same instructions -
// made decode_32k's step 0.4-0.6 us slower (measured: the step returned to
// its earlier time once the wide kernels moved to a separate code object).
// Arguments pass as the bytes of this file's FusedSelect and AttnParams.
extern "C" __attribute__((visibility("hidden"))) int qsa_attn_launch_fused_wide(
    const void* select, size_t select_bytes, const void* params, size_t params_bytes,
    unsigned grid_x, unsigned grid_y, unsigned grid_z, int head_dim, int nkv, hipStream_t stream);

namespace qsa {
namespace {

constexpr int kTile = 32;
constexpr float kInitMax = -1.0e20f;  // finite running-max seed (ops/qsa.py:173)
constexpr int kMergeChunk = 8;        // split partials a merge thread loads at once
constexpr int kCUs = 256;             // compute units of an MI355X

struct AttnParams {
  const uint16_t* q;
  int64_t q_row, q_head;  // elements
  const char* k;
  const char* v;
  int64_t kb, kt, kh;  // bytes
  int64_t vb, vt, vh;  // bytes
  int num_blocks;
  int page_size;
  FastDiv page_div;
  // Buffer addressing (token-major K/V views spanning under 4 GB): the byte
  // range of one kv head's rows from that head's base ((num_slots - 1) x
  // token stride + one row) and the token strides, 32-bit.
  uint32_t k_bytes, v_bytes;
  uint32_t kt32, vt32;
  int num_slots;
  const int32_t* indices;
  int64_t idx_row;
  int width;
  const int32_t* table;
  int64_t table_row;
  int table_width;
  int num_requests;
  const int32_t* token_to_req;
  const int32_t* valid_counts;
  uint16_t* out;
  int64_t out_row, out_head;  // elements
  const uint16_t* gate;
  int64_t g_row, g_head, g_dim;  // elements
  float* part_out;
  float* part_lse;
  int rows;
  int num_q_heads;
  int group;
  int heads_per_wave;
  int num_splits;
  int physical;
  float scale_log2;
};

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

#define QSA_SCHED_FENCE() __builtin_amdgcn_sched_barrier(0)

// Validated slot (page * page_size + offset) of a physical index value, or
// -1 (ops/qsa.py:186-212).
__device__ __forceinline__ int physical_slot(const AttnParams& p, int tok) {
  const int lp = p.page_div.div(max(tok, 0));
  return (tok >= 0 && lp < p.num_blocks) ? tok : -1;
}

// Logical indices in two steps (ops/qsa.py:186-212), so the block-table loads
// can be issued a whole tile ahead of the K/V loads that need them: the table
// entries of a tile's index values (unconditional loads, the zero block where
// an entry is not mapped), then the validated slots.
__device__ __forceinline__ int table_page(const AttnParams& p, const int32_t* trow, bool req_ok,
                                          int tok) {
  const int lp = p.page_div.div(max(tok, 0));
  const bool mapped = tok >= 0 && req_ok && lp < p.table_width;
  return *(mapped ? trow + lp : reinterpret_cast<const int32_t*>(g_qsa_zero_rows));
}
__device__ __forceinline__ int logical_slot(const AttnParams& p, bool req_ok, int tok, int page) {
  const int lp = p.page_div.div(max(tok, 0));
  const bool mapped = tok >= 0 && req_ok && lp < p.table_width;
  return (mapped && page >= 0 && page < p.num_blocks) ? page * p.page_size + (tok - lp * p.page_size)
                                                      : -1;
}

// Byte offset of a validated slot's row in a cache with (block, token) strides.
__device__ __forceinline__ int64_t slot_offset(const AttnParams& p, int slot, int64_t sb,
                                               int64_t st) {
  const int page = p.page_div.div(slot);
  return (int64_t)page * sb + (int64_t)(slot - page * p.page_size) * st;
}

// Buffer addressing. A token-major view (block stride = page_size x token
// stride) puts slot s's row of kv head v at s x token_stride from the head's
// base, so one buffer resource per kv head and a 32-bit byte offset address
// every row: one multiply per slot instead of a page division and 64-bit
// arithmetic. An invalid slot gets an offset past every resource's range,
// where the hardware's range check returns zeros (the zero block's role on
// the 64-bit path).
constexpr uint32_t kOobOffset = 0xFFFFF000u;  // + lane and step offsets stays past any range
constexpr uint32_t kMaxBufferBytes = 0xFFFF0000u;
constexpr int kRawBufferWord3 = 0x00020000;  // raw (unformatted) dword access

template <int NKV>
struct KVBuffers {
  __amdgpu_buffer_rsrc_t k[NKV];
  __amdgpu_buffer_rsrc_t v[NKV];
};

template <int NKV>
__device__ __forceinline__ KVBuffers<NKV> make_kv_buffers(const AttnParams& p, int kv0) {
  KVBuffers<NKV> b;
#pragma unroll
  for (int v = 0; v < NKV; ++v) {
    const uint32_t kh = (uint32_t)((kv0 + v) * p.kh);
    const uint32_t vh = (uint32_t)((kv0 + v) * p.vh);
    b.k[v] = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(p.k) + kh, (short)0,
                                               (int)p.k_bytes, kRawBufferWord3);
    b.v[v] = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(p.v) + vh, (short)0,
                                               (int)p.v_bytes, kRawBufferWord3);
  }
  return b;
}

// A physical index value is a valid slot iff it lies in the cache.
__device__ __forceinline__ int physical_slot_flat(const AttnParams& p, int tok) {
  return (tok >= 0 && tok < p.num_slots) ? tok : -1;
}

template <int D>
struct VRow;
template <>
struct VRow<128> {
  typedef u32x4 type;
  static __device__ __forceinline__ type load(const char* ptr) { return load_u32x4(ptr); }
};
template <>
struct VRow<64> {
  typedef u32x2 type;
  static __device__ __forceinline__ type load(const char* ptr) { return load_u32x2(ptr); }
};

// One tile's operands in registers. K and V rows are loaded alike: lane
// (n, g) loads dims DPL n .. DPL n + DPL - 1 of tokens 16 (i / 4) + 4 g + i % 4
// (four tokens' whole rows per load instruction; a load of 16 tokens x 64 B
// instead, the MFMA layout, measured half the L2 throughput). K then moves
// through the wave's LDS region into the MFMA A layout: lane (n, g) holds
// dims 32 s + 8 g .. + 7 of token 16 u + n.
template <int D, int NKV>
struct TileK {
  u32x4 r[NKV][2][D / 32];
};
template <int D, int NKV>
struct TileKRows {
  typename VRow<D>::type r[NKV][8];
};
template <int D, int NKV>
struct TileV {
  typename VRow<D>::type r[NKV][8];
  uint32_t mask;  // bit i: token slot i is valid
};

__device__ __forceinline__ int k_col(int tile, int u, int n) { return tile * kTile + 16 * u + n; }

// Raw index entries of a tile's K tokens 16 u + n. Every entry is loaded
// unconditionally (columns past the valid count or the split read the zero
// block) with its validity in `ok`, applied only when the entry is used: a
// skipped load would make the compiler drain every outstanding load at the
// first use instead of waiting for these loads alone.
struct TileIdx {
  int k[2];
  uint32_t ok;  // bit u: k[u]
  __device__ __forceinline__ int key(int u) const { return (ok >> u) & 1u ? k[u] : -1; }
};
// LDS: irow is a row of entries in LDS (the fused selection's), read at
// column 0 where an entry is not valid.
template <bool LDS>
__device__ __forceinline__ void load_tile_idx(const int32_t* irow, int tile, int t_end,
                                              int n_valid, int n, TileIdx& r) {
  const int32_t* zero = reinterpret_cast<const int32_t*>(g_qsa_zero_rows);
  const bool live = tile < t_end;
  r.ok = 0;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int col = k_col(tile, u, n);
    const bool ok = live && col < n_valid;
    if constexpr (LDS) r.k[u] = irow[ok ? col : 0];
    else r.k[u] = *(ok ? irow + col : zero);
    r.ok |= (uint32_t)ok << u;
  }
}

// Slots of the lane's V tokens 16 (i / 4) + 4 g + i % 4: each is the K token
// 16 u + n of lane 16 g + n with u = i / 4, n = 4 g + i % 4, in the same row
// of 16 lanes.
__device__ __forceinline__ void v_slots_from_k(const int (&ks)[2], int g, int (&vs)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i)
    vs[i] = __builtin_amdgcn_ds_bpermute((20 * g + (i & 3)) * 4, ks[i >> 2]);
}

// K in the MFMA A layout straight from memory (lane (n, g): dims 32 s + 8 g
// .. + 7 of token 16 u + n; 16 tokens x 64 B per load instruction). Used for
// logical (prefill) rows with D = 64, where it measured faster than staging K
// through registers and LDS; D = 128 logical rows load whole rows straight
// into LDS (dma_k), physical (decode) rows load whole rows and stage them
// (stage_k).
template <int D, int NKV>
__device__ __forceinline__ void issue_k_direct(const AttnParams& p, const int (&slot)[2],
                                               const int64_t (&khead)[NKV], int g,
                                               TileK<D, NKV>& K) {
  const char* zero = reinterpret_cast<const char*>(g_qsa_zero_rows);
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int64_t off = slot[u] >= 0 ? slot_offset(p, slot[u], p.kb, p.kt) : 0;
#pragma unroll
    for (int v = 0; v < NKV; ++v) {
      const char* base = slot[u] >= 0 ? p.k + off + khead[v] : zero;
#pragma unroll
      for (int s = 0; s < D / 32; ++s) K.r[v][u][s] = load_u32x4(base + (32 * s + 8 * g) * 2);
    }
  }
}

template <int D, int NKV>
__device__ __forceinline__ void issue_k(const AttnParams& p, const int (&slot)[8],
                                        const int64_t (&khead)[NKV], int n, TileKRows<D, NKV>& K) {
  constexpr int DPL = D / 16;
  const char* zero = reinterpret_cast<const char*>(g_qsa_zero_rows);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t off = slot[i] >= 0 ? slot_offset(p, slot[i], p.kb, p.kt) : 0;
#pragma unroll
    for (int v = 0; v < NKV; ++v) {
      const char* base = slot[i] >= 0 ? p.k + off + khead[v] : zero;
      K.r[v][i] = VRow<D>::load(base + DPL * n * 2);
    }
  }
}

template <int D, int NKV>
__device__ __forceinline__ void issue_v(const AttnParams& p, const int (&slot)[8],
                                        const int64_t (&vhead)[NKV], int n, TileV<D, NKV>& V) {
  constexpr int DPL = D / 16;
  const char* zero = reinterpret_cast<const char*>(g_qsa_zero_rows);
  V.mask = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    V.mask |= slot[i] >= 0 ? (1u << i) : 0u;
    const int64_t off = slot[i] >= 0 ? slot_offset(p, slot[i], p.vb, p.vt) : 0;
#pragma unroll
    for (int v = 0; v < NKV; ++v) {
      const char* base = slot[i] >= 0 ? p.v + off + vhead[v] : zero;
      V.r[v][i] = VRow<D>::load(base + DPL * n * 2);
    }
  }
}

template <int D>
struct VRowBuf;
template <>
struct VRowBuf<128> {
  static __device__ __forceinline__ u32x4 load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
  }
};
template <>
struct VRowBuf<64> {
  static __device__ __forceinline__ u32x2 load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
  }
};

template <int D, int NKV>
__device__ __forceinline__ void issue_k_direct(const AttnParams& p, const KVBuffers<NKV>& b,
                                               const int (&slot)[2], int g, TileK<D, NKV>& K) {
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const uint32_t off = slot[u] >= 0 ? (uint32_t)slot[u] * p.kt32 + 16 * g : kOobOffset;
#pragma unroll
    for (int v = 0; v < NKV; ++v)
#pragma unroll
      for (int s = 0; s < D / 32; ++s)
        K.r[v][u][s] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(b.k[v], off + 64 * s, 0, 0));
  }
}

template <int D, int NKV>
__device__ __forceinline__ void issue_k(const AttnParams& p, const KVBuffers<NKV>& b,
                                        const int (&slot)[8], int n, TileKRows<D, NKV>& K) {
  constexpr int DPL = D / 16;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t off = slot[i] >= 0 ? (uint32_t)slot[i] * p.kt32 + DPL * n * 2 : kOobOffset;
#pragma unroll
    for (int v = 0; v < NKV; ++v) K.r[v][i] = VRowBuf<D>::load(b.k[v], off);
  }
}

// K rows -> the wave's LDS region -> MFMA A layout. The region holds (kv v,
// token) rows of U = D / 8 16-byte units, the unit index XOR-swizzled by the
// token, so both the row writes (16 lanes per row) and the A-layout reads
// (16 tokens per unit position) are conflict-free. A wave's LDS accesses
// complete in order, so the reads see the writes.
//
// Every address is a per-lane byte offset plus a compile-time row offset (the
// DS instruction's immediate): a write of token 16 (i / 4) + 4 g + a lands at
// wr[a] + (v kTile + 16 (i / 4)) U 16, a read of token 16 u + n, unit 4 s + g
// at rd[s] + (v kTile + 16 u) U 16 (16 (i / 4) and 16 u leave the token's
// residue mod U unchanged, which is all the swizzle depends on).
template <int D>
struct KStageLanes {
  uint32_t wr[4];
  uint32_t rd[D / 32];
};
template <int D>
__device__ __forceinline__ KStageLanes<D> k_stage_lanes(uint32_t region, int n, int g) {
  constexpr int U = D / 8;
  KStageLanes<D> l;
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int tok = 4 * g + a;
    l.wr[a] = region + (uint32_t)(tok * U * 16) +
              (D == 128 ? (uint32_t)((n ^ (tok % U)) * 16)
                        : (uint32_t)(((n >> 1) ^ (tok % U)) * 16 + (n & 1) * 8));
  }
#pragma unroll
  for (int s2 = 0; s2 < D / 32; ++s2)
    l.rd[s2] = region + (uint32_t)((n * U + ((4 * s2 + g) ^ (n % U))) * 16);
  return l;
}

template <int D, int NKV>
__device__ __forceinline__ void stage_k(char* lds, const KStageLanes<D>& l,
                                        const TileKRows<D, NKV>& KR, TileK<D, NKV>& K) {
  constexpr int U = D / 8;
#pragma unroll
  for (int v = 0; v < NKV; ++v)
#pragma unroll
    for (int i = 0; i < 8; ++i)
      *reinterpret_cast<typename VRow<D>::type*>(
          lds + l.wr[i & 3] + (v * kTile + 16 * (i >> 2)) * U * 16) = KR.r[v][i];
#pragma unroll
  for (int v = 0; v < NKV; ++v)
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int s2 = 0; s2 < D / 32; ++s2)
        K.r[v][u][s2] = *reinterpret_cast<const u32x4*>(lds + l.rd[s2] +
                                                        (v * kTile + 16 * u) * U * 16);
}

// K rows straight into the wave's LDS region (global_load_lds_dwordx4: lane l
// of an instruction writes its 16 bytes at the destination + 16 l), for
// logical (prefill) rows with D = 128. Instruction (v, i) covers the four
// tokens 16 (i / 4) + 4 g + i % 4 of V's load pattern, one 256 B row per
// 16-lane row g, into the 1 KB block v 8 KB + i KB; lane (n, g) loads the row's
// 16-byte unit n ^ (token % 16), so unit c of token 16 u + m sits at position
// c ^ m of its row and the A-layout reads (16 tokens per unit position) are
// conflict-free. The data never passes through VGPRs; the wave waits for it
// (vmcnt) only when it reads the block back.
constexpr int kDmaKBlockBytes = 1024;

// s_waitcnt immediate that waits for the vector-memory counter alone (gfx9
// encoding: vmcnt in bits 3:0 and 15:14, expcnt and lgkmcnt at their maxima).
constexpr int vmcnt_only(int n) { return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14); }

template <int D, int NKV>
__device__ __forceinline__ void dma_k(const AttnParams& p, const int (&slot)[8],
                                      const int64_t (&khead)[NKV], int n, int g, char* region) {
  static_assert(D == 128, "one 256 B row per 16 lanes");
  const char* zero = reinterpret_cast<const char*>(g_qsa_zero_rows);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t off = slot[i] >= 0 ? slot_offset(p, slot[i], p.kb, p.kt) : 0;
    const int unit = 16 * (n ^ (4 * g + (i & 3)));
#pragma unroll
    for (int v = 0; v < NKV; ++v) {
      const char* src = (slot[i] >= 0 ? p.k + off + khead[v] : zero) + unit;
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void*)src,
          (__attribute__((address_space(3))) void*)(region + (v * 8 + i) * kDmaKBlockBytes), 16,
          0, 0);
    }
  }
}

// The A layout from a region dma_k filled: lane (n, g) reads unit 4 s + g of
// token 16 u + n, written by instruction 4 u + n % 4 in row n / 4.
template <int D, int NKV>
__device__ __forceinline__ void read_k_dma(const char* region, int n, int g, TileK<D, NKV>& K) {
  const char* lane_base = region + (n & 3) * kDmaKBlockBytes + (n >> 2) * 256;
#pragma unroll
  for (int v = 0; v < NKV; ++v)
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int s = 0; s < D / 32; ++s)
        K.r[v][u][s] = *reinterpret_cast<const u32x4*>(
            lane_base + (v * 8 + 4 * u) * kDmaKBlockBytes + 16 * ((4 * s + g) ^ n));
}

template <int D, int NKV>
__device__ __forceinline__ void issue_v(const AttnParams& p, const KVBuffers<NKV>& b,
                                        const int (&slot)[8], int n, TileV<D, NKV>& V) {
  constexpr int DPL = D / 16;
  V.mask = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    V.mask |= slot[i] >= 0 ? (1u << i) : 0u;
    const uint32_t off = slot[i] >= 0 ? (uint32_t)slot[i] * p.vt32 + DPL * n * 2 : kOobOffset;
#pragma unroll
    for (int v = 0; v < NKV; ++v) V.r[v][i] = VRowBuf<D>::load(b.v[v], off);
  }
}

// S^T = K_tile Q^T, then the online-softmax update of head n; returns P^T (the
// lane's 8 token numerators) as packed bf16 pairs. Each kv head's scores are
// computed for all 16 head columns and every lane keeps its own head's kv.
template <int D, int NKV>
__device__ __forceinline__ u32x4 qk_softmax(const AttnParams& p, const TileK<D, NKV>& K,
                                            const bf16x8 (&bq)[D / 32], int vslot, uint32_t mask,
                                            float& m_run, float& l_run, f32x4 (&oacc)[D / 16]) {
  f32x4 sacc[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    f32x4 sel = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int v = 0; v < NKV; ++v) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < D / 32; ++s)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, K.r[v][u][s]),
                                                      bq[s], acc, 0, 0, 0);
      sel = vslot == v ? acc : sel;
    }
    sacc[u] = sel;
  }
  // Lane holds S[token 16 u + 4 g + r][head n] in sacc[u][r] = token slot 4 u + r.
  float sc[8];
  float tmax = -INFINITY;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float x = sacc[i >> 2][i & 3] * p.scale_log2;
    sc[i] = (mask >> i) & 1u ? x : -INFINITY;
    tmax = fmaxf(tmax, sc[i]);
  }
  tmax = fmaxf(tmax, shfl_xor_f(tmax, 16));
  tmax = fmaxf(tmax, shfl_xor_f(tmax, 32));
  const float m_new = fmaxf(m_run, tmax);
  const float alpha = fast_exp2(m_run - m_new);
  float lsum = 0.0f;
  float pv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    pv[i] = fast_exp2(sc[i] - m_new);
    lsum += pv[i];
  }
  l_run = l_run * alpha + lsum;
  m_run = m_new;
#pragma unroll
  for (int j = 0; j < D / 16; ++j) oacc[j] *= alpha;
  u32x4 praw;
  praw[0] = pack_bf16x2(pv[0], pv[1]);
  praw[1] = pack_bf16x2(pv[2], pv[3]);
  praw[2] = pack_bf16x2(pv[4], pv[5]);
  praw[3] = pack_bf16x2(pv[6], pv[7]);
  return praw;
}

// O^T += V_tile^T P^T, the lane's 8x8 V blocks transposed by v_perm_b32.
template <int D, int NKV>
__device__ __forceinline__ void pv_mfma(const TileV<D, NKV>& V, u32x4 praw, int vslot,
                                        f32x4 (&oacc)[D / 16]) {
#pragma unroll
  for (int v = 0; v < NKV; ++v) {
    const u32x4 pm = (vslot == v) ? praw : u32x4{0u, 0u, 0u, 0u};
    const bf16x8 bp = __builtin_bit_cast(bf16x8, pm);
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
      const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
      u32x4 a;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        a[q] = perm_b32(V.r[v][2 * q + 1][j >> 1], V.r[v][2 * q][j >> 1], sel);
      oacc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), bp,
                                                        oacc[j], 0, 0, 0);
    }
  }
}

// LDS of one attention workgroup: each wave's K staging region (physical
// rows, or the direct loads of logical rows with D = 128), which the waves'
// partial outputs reuse for the combine after the tile loop, and the waves'
// running maxima and sums.
template <int D, int NKV, int WAVES, bool PHYSICAL>
struct AttnLds {
  static constexpr bool kDmaK = !PHYSICAL && D == 128;
  static constexpr int kStageUnits = (PHYSICAL || kDmaK) ? NKV * kTile * (D / 8) : 0;
  static constexpr int kStageBytes = WAVES * kStageUnits * 16;
  static constexpr int kCombineBytes = WAVES * 16 * (D + 4) * 4;
  static constexpr int kBufBytes = kStageBytes > kCombineBytes ? kStageBytes : kCombineBytes;
};

// One workgroup's share of the attention: row `row`, split `split` of
// p.num_splits, head group `hg`. Index entries come from global memory
// (p.indices, p.valid_counts) or, with LDS_IDX, from a row of n_valid_lds
// entries in LDS at irow_lds.
template <int D, int NKV, int WAVES, bool PHYSICAL, bool BUF, bool LDS_IDX>
__device__ __forceinline__ void attend(const AttnParams& p, int row, int split, int hg,
                                       const int32_t* irow_lds, int n_valid_lds, char* s_lds,
                                       float (*s_m)[16], float (*s_l)[16]) {
  constexpr int DPL = D / 16;  // V dims per lane = P.V MFMAs per kv slot
  constexpr int KS = D / 32;   // K steps of the Q.K MFMA

  // Logical rows with D = 128 load K rows into LDS directly (dma_k).
  constexpr bool DMA_K = AttnLds<D, NKV, WAVES, PHYSICAL>::kDmaK;
  constexpr int kStageUnits = AttnLds<D, NKV, WAVES, PHYSICAL>::kStageUnits;
  float(*s_o)[16][D + 4] = reinterpret_cast<float(*)[16][D + 4]>(s_lds);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4;
  const int n = lane & 15;

  const int head0 = hg * p.heads_per_wave;
  const int kv0 = head0 / p.group;
  const bool head_ok = n < p.heads_per_wave;
  const int qh = head0 + n;
  const int vslot = head_ok ? qh / p.group - kv0 : -1;

  // Q^T as the B operand: lane holds Q[qh][32 s + 8 g .. +7].
  bf16x8 bq[KS];
  {
    const uint16_t* qrow = p.q + (int64_t)row * p.q_row + (int64_t)(head_ok ? qh : 0) * p.q_head;
    const void* zero = g_qsa_zero_rows;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      bq[s] = __builtin_bit_cast(
          bf16x8, load_u32x4(head_ok ? (const void*)(qrow + 32 * s + 8 * g) : zero));
  }

  int n_valid = p.width;
  if constexpr (LDS_IDX) n_valid = max(0, min(n_valid_lds, p.width));
  else if (p.valid_counts) n_valid = max(0, min(p.valid_counts[row], p.width));
  const int req = p.token_to_req[row];
  const bool req_ok = req >= 0 && req < p.num_requests;
  const int32_t* trow = p.table + (int64_t)(req_ok ? req : 0) * p.table_row;
  const int32_t* irow = LDS_IDX ? irow_lds : p.indices + (int64_t)row * p.idx_row;
  const int tiles = (n_valid + kTile - 1) / kTile;
  const int t_begin = (int)((int64_t)split * tiles / p.num_splits);
  const int t_end = (int)((int64_t)(split + 1) * tiles / p.num_splits);

  int64_t khead[NKV], vhead[NKV];
#pragma unroll
  for (int v = 0; v < NKV; ++v) {
    khead[v] = (int64_t)(kv0 + v) * p.kh;
    vhead[v] = (int64_t)(kv0 + v) * p.vh;
  }
  KVBuffers<NKV> kvb;
  if constexpr (BUF) kvb = make_kv_buffers<NKV>(p, kv0);
  // K/V loads and physical slot validation of the chosen addressing.
  auto load_k = [&](const int (&slot)[8], TileKRows<D, NKV>& K) {
    if constexpr (BUF) issue_k<D, NKV>(p, kvb, slot, n, K);
    else issue_k<D, NKV>(p, slot, khead, n, K);
  };
  const KStageLanes<D> k_lanes = k_stage_lanes<D>((uint32_t)(wave * kStageUnits * 16), n, g);  // physical rows
  auto load_k_direct = [&](const int (&slot)[2], TileK<D, NKV>& K) {
    if constexpr (BUF) issue_k_direct<D, NKV>(p, kvb, slot, g, K);
    else issue_k_direct<D, NKV>(p, slot, khead, g, K);
  };
  auto load_v = [&](const int (&slot)[8], TileV<D, NKV>& V) {
    if constexpr (BUF) issue_v<D, NKV>(p, kvb, slot, n, V);
    else issue_v<D, NKV>(p, slot, vhead, n, V);
  };
  auto phys = [&](int tok) { return BUF ? physical_slot_flat(p, tok) : physical_slot(p, tok); };

  float m_run = kInitMax;
  float l_run = 0.0f;
  f32x4 oacc[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) oacc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  int t = t_begin + wave;
  if constexpr (DMA_K) {
    if (t < t_end) {
    // As the three-stage loop below, with K rows loaded into the wave's LDS
    // region: per trip, K(t) is read back (waiting for its loads only), then
    // K(t+W) is issued into the same region, table(t+2W), index(t+3W),
    // V(t+W). The slots of K(t+W) come from lanes' ds_bpermute, which
    // completes after the reads of K(t) (LDS operations complete in order),
    // so the new rows never overwrite rows not yet read.
    char* kregion = s_lds + wave * kStageUnits * 16;
    TileIdx ia, ib;
    int pa[2];
    int ks[2], vs[8];
    TileK<D, NKV> K;
    TileV<D, NKV> V;
    load_tile_idx<LDS_IDX>(irow, t, t_end, n_valid, n, ia);
#pragma unroll
    for (int u = 0; u < 2; ++u) pa[u] = table_page(p, trow, req_ok, ia.key(u));
#pragma unroll
    for (int u = 0; u < 2; ++u) ks[u] = logical_slot(p, req_ok, ia.key(u), pa[u]);
    v_slots_from_k(ks, g, vs);
    load_tile_idx<LDS_IDX>(irow, t + WAVES, t_end, n_valid, n, ia);
    QSA_SCHED_FENCE();
    dma_k<D, NKV>(p, vs, khead, n, g, kregion);
    QSA_SCHED_FENCE();
#pragma unroll
    for (int u = 0; u < 2; ++u) pa[u] = table_page(p, trow, req_ok, ia.key(u));
    QSA_SCHED_FENCE();
    load_tile_idx<LDS_IDX>(irow, t + 2 * WAVES, t_end, n_valid, n, ib);
    QSA_SCHED_FENCE();
    load_v(vs, V);
    QSA_SCHED_FENCE();
    for (; t < t_end; t += WAVES) {
      // K(t) has landed once at most the loads issued after it (table 2,
      // index 2, V 8 NKV) are outstanding; the compiler does not order LDS
      // reads after direct loads into LDS by itself.
      __builtin_amdgcn_s_waitcnt(vmcnt_only(4 + 8 * NKV));
      read_k_dma<D, NKV>(kregion, n, g, K);
      QSA_SCHED_FENCE();
#pragma unroll
      for (int u = 0; u < 2; ++u) ks[u] = logical_slot(p, req_ok, ia.key(u), pa[u]);
      v_slots_from_k(ks, g, vs);
      dma_k<D, NKV>(p, vs, khead, n, g, kregion);
      QSA_SCHED_FENCE();
      const u32x4 praw = qk_softmax<D, NKV>(p, K, bq, vslot, V.mask, m_run, l_run, oacc);
      QSA_SCHED_FENCE();
      pv_mfma<D, NKV>(V, praw, vslot, oacc);
      QSA_SCHED_FENCE();
#pragma unroll
      for (int u = 0; u < 2; ++u) pa[u] = table_page(p, trow, req_ok, ib.key(u));
      ia = ib;
      QSA_SCHED_FENCE();
      load_tile_idx<LDS_IDX>(irow, t + 3 * WAVES, t_end, n_valid, n, ib);
      QSA_SCHED_FENCE();
      load_v(vs, V);
      QSA_SCHED_FENCE();
    }
    // The last trip's K loads (of the tile past the split: the zero block)
    // land in LDS that the combine reuses.
    __builtin_amdgcn_s_waitcnt(0);
    }
  } else if constexpr (!PHYSICAL) {
    if (t < t_end) {
    // Three stages: index entries of t+3W, table entries of t+2W, K/V of t+W
    // are in flight while tile t computes. Issue order per trip: K(t+W),
    // table(t+2W), index(t+3W), V(t+W); each wait is for the oldest group.
    TileIdx ia, ib;  // index entries of t+W (table entries in flight) and of t+2W
    int pa[2];       // table entries of t+W
    int ks[2], vs[8];
    TileK<D, NKV> K;
    TileV<D, NKV> V;
    load_tile_idx<LDS_IDX>(irow, t, t_end, n_valid, n, ia);
#pragma unroll
    for (int u = 0; u < 2; ++u) pa[u] = table_page(p, trow, req_ok, ia.key(u));
#pragma unroll
    for (int u = 0; u < 2; ++u) ks[u] = logical_slot(p, req_ok, ia.key(u), pa[u]);
    v_slots_from_k(ks, g, vs);
    load_tile_idx<LDS_IDX>(irow, t + WAVES, t_end, n_valid, n, ia);
    QSA_SCHED_FENCE();
    load_k_direct(ks, K);
    QSA_SCHED_FENCE();
#pragma unroll
    for (int u = 0; u < 2; ++u) pa[u] = table_page(p, trow, req_ok, ia.key(u));
    QSA_SCHED_FENCE();
    load_tile_idx<LDS_IDX>(irow, t + 2 * WAVES, t_end, n_valid, n, ib);
    QSA_SCHED_FENCE();
    load_v(vs, V);
    QSA_SCHED_FENCE();
    for (; t < t_end; t += WAVES) {
      const u32x4 praw = qk_softmax<D, NKV>(p, K, bq, vslot, V.mask, m_run, l_run, oacc);
      QSA_SCHED_FENCE();
#pragma unroll
      for (int u = 0; u < 2; ++u) ks[u] = logical_slot(p, req_ok, ia.key(u), pa[u]);
      load_k_direct(ks, K);
      QSA_SCHED_FENCE();
      pv_mfma<D, NKV>(V, praw, vslot, oacc);
      QSA_SCHED_FENCE();
#pragma unroll
      for (int u = 0; u < 2; ++u) pa[u] = table_page(p, trow, req_ok, ib.key(u));
      ia = ib;  // arrived: its table entries were just addressed from it
      QSA_SCHED_FENCE();
      load_tile_idx<LDS_IDX>(irow, t + 3 * WAVES, t_end, n_valid, n, ib);
      QSA_SCHED_FENCE();
      v_slots_from_k(ks, g, vs);
      load_v(vs, V);
      QSA_SCHED_FENCE();
    }
    }
  } else {
    if (t < t_end) {
    TileIdx idx;
    int ks[2], vs[8];
    TileK<D, NKV> K;
    TileKRows<D, NKV> KR;
    TileV<D, NKV> V;
    // Prologue, in issue order: K(t), index entries of t+W, V(t).
    load_tile_idx<LDS_IDX>(irow, t, t_end, n_valid, n, idx);
#pragma unroll
    for (int u = 0; u < 2; ++u) ks[u] = phys(idx.key(u));
    v_slots_from_k(ks, g, vs);
    load_k(vs, KR);
    QSA_SCHED_FENCE();
    load_tile_idx<LDS_IDX>(irow, t + WAVES, t_end, n_valid, n, idx);
    QSA_SCHED_FENCE();
    load_v(vs, V);
    QSA_SCHED_FENCE();
    // The next tile's loads are issued even on the last trip (its slots are
    // then all invalid and read the zero block): loads under a branch would
    // make the compiler's wait counts assume the branch not taken, so P.V(t)
    // would also wait for K(t+W).
    for (; t < t_end; t += WAVES) {
      stage_k<D, NKV>(s_lds, k_lanes, KR, K);
      const u32x4 praw = qk_softmax<D, NKV>(p, K, bq, vslot, V.mask, m_run, l_run, oacc);
      QSA_SCHED_FENCE();
#pragma unroll
      for (int u = 0; u < 2; ++u) ks[u] = phys(idx.key(u));
      v_slots_from_k(ks, g, vs);
      load_k(vs, KR);
      QSA_SCHED_FENCE();
      pv_mfma<D, NKV>(V, praw, vslot, oacc);
      QSA_SCHED_FENCE();
      load_tile_idx<LDS_IDX>(irow, t + 2 * WAVES, t_end, n_valid, n, idx);
      QSA_SCHED_FENCE();
      load_v(vs, V);
      QSA_SCHED_FENCE();
    }
    }
  }

  // Row sums are lane-partial (each lane summed its own tokens).
  l_run += shfl_xor_f(l_run, 16);
  l_run += shfl_xor_f(l_run, 32);

  // s_o shares LDS with the other waves' K staging regions.
  if constexpr (PHYSICAL || DMA_K) __syncthreads();
  // oacc[j][r] = O[head n][DPL * (4 g + r) + j].
#pragma unroll
  for (int j = 0; j < DPL; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) s_o[wave][n][DPL * (4 * g + r) + j] = oacc[j][r];
  if (g == 0) {
    s_m[wave][n] = m_run;
    s_l[wave][n] = l_run;
  }
  __syncthreads();

  // Thread t < 256 finalises head t / 16, dims [(t % 16) * DPL, +DPL).
  const int h = threadIdx.x >> 4;
  const int d0 = (threadIdx.x & 15) * DPL;
  if (threadIdx.x >= 256 || h >= p.heads_per_wave) return;
  const int head = head0 + h;
  float mw[WAVES];
  float mx = kInitMax, lsum = 0.0f;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) {
    mw[w] = s_m[w][h];
    mx = fmaxf(mx, mw[w]);
  }
  float o[DPL];
#pragma unroll
  for (int d = 0; d < DPL; ++d) o[d] = 0.0f;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) {
    const float wt = fast_exp2(mw[w] - mx);
    lsum += wt * s_l[w][h];
#pragma unroll
    for (int d = 0; d < DPL; ++d) o[d] += wt * s_o[w][h][d0 + d];
  }
  const float inv = lsum > 0.0f ? 1.0f / fmaxf(lsum, 1.0e-20f) : 0.0f;
#pragma unroll
  for (int d = 0; d < DPL; ++d) o[d] *= inv;

  if (p.num_splits > 1) {
    // Normalised fp32 partial + log2-LSE for the merge kernel (ops/qsa.py:278-303).
    const int64_t prow = ((int64_t)split * p.rows + row) * p.num_q_heads + head;
    float* po = p.part_out + prow * D + d0;
#pragma unroll
    for (int d = 0; d < DPL; ++d) po[d] = o[d];
    if ((threadIdx.x & 15) == 0)
      p.part_lse[prow] = lsum > 0.0f ? mx + __log2f(fmaxf(lsum, 1.0e-20f)) : -INFINITY;
    return;
  }

  uint16_t* optr = p.out + (int64_t)row * p.out_row + (int64_t)head * p.out_head + d0;
  const uint16_t* gptr = p.gate ? p.gate + (int64_t)row * p.g_row + (int64_t)head * p.g_head : nullptr;
#pragma unroll
  for (int d = 0; d < DPL; d += 2) {
    float a = o[d], b = o[d + 1];
    if (gptr) {
      // bf16(o) * sigmoid(gate) (ops/qsa.py:257-269).
      const uint32_t ob = pack_bf16x2(a, b);
      const float ga = bf16_lo((uint32_t)gptr[(int64_t)(d0 + d) * p.g_dim]);
      const float gb = bf16_lo((uint32_t)gptr[(int64_t)(d0 + d + 1) * p.g_dim]);
      a = bf16_lo(ob) * sigmoidf_(ga);
      b = bf16_hi(ob) * sigmoidf_(gb);
    }
    *reinterpret_cast<uint32_t*>(optr + d) = pack_bf16x2(a, b);
  }
}

// Two waves per SIMD wherever the registers allow it without spilling.
template <int D, int NKV, int WAVES, bool PHYSICAL, bool BUF>
__global__ __launch_bounds__(64 * WAVES)
__attribute__((amdgpu_waves_per_eu(D == 128 && NKV == 4 ? 1 : 2)))
void sparse_attn_kernel(const AttnParams p) {
  __shared__ __attribute__((aligned(16))) char s_lds[AttnLds<D, NKV, WAVES, PHYSICAL>::kBufBytes];
  __shared__ float s_m[WAVES][16];
  __shared__ float s_l[WAVES][16];
  attend<D, NKV, WAVES, PHYSICAL, BUF, false>(p, blockIdx.x, blockIdx.y, blockIdx.z, nullptr, 0,
                                              s_lds, s_m, s_l);
}

// Decode selection fused with the attention (physical slots, 8-wave
// workgroups). Every workgroup of a row first selects the row itself, with the
// top-k kernel's whole-row code (topk_device.h) on all of the workgroup's
// threads, and writes the expanded row into LDS instead of global memory; its
// attention then reads its index entries from LDS. The row's selection is
// computed once per workgroup of the row (splits x head groups copies of a
// row of at most 2048 columns, a few KB each), which removes the top-k launch,
// its boundary with the attention, and the attention's first index round
// trip. Workgroup (row, 0, 0) also writes the expanded row and its count for
// the caller, after its attention, so no store sits ahead of its K/V loads in
// the wave's in-order memory counter.
constexpr int kFusedMaxWidth = 4160;  // LDS-resident expanded row (4096 + a causal tail)

struct FusedSelect {
  const float* scores;
  int64_t score_row_stride;
  const int32_t* lengths;
  int cols;
  int topk;
  ExpandMeta meta;  // physical expansion into LDS: out_col_stride 1, no counts
  int32_t* indices;  // the caller's copy of the expanded rows
  int64_t indices_row_stride;
  int32_t* counts;
};

template <int THREADS, int ITEMS>
struct FusedTopkLds {
  TopkShared<THREADS> sh;
  alignas(16) TopkStage<THREADS, ITEMS, true> st;
};

// Selection LDS of a wide buffer's long rows (select_wide_row).
struct FusedWideLds {
  TopkShared<kWideThreads> sh;
  alignas(16) uint32_t stage[kWideThreads * 32 * 2];
};

// WIDE 1: a logits buffer wider than 8192 columns (a decode batch in a wide
// width class, whose rows are usually much shorter than the buffer). As
// topk_adaptive_kernel does, every workgroup issues the loads of the row's
// first 2048 columns in the 512 x 4 shape before the row's length arrives;
// a row of at most 2048 keys is then selected from them, a longer one by
// select_wide_row (up to 32768 keys, slower than the top-k launch's 1024
// threads, but a row that long is rare in such a class).
// WIDE 2: a buffer of 2049 to 8192 columns, whose rows are often longer than
// 2048 keys: the loads of every column go out before the length arrives (16
// per thread; element i * 512 + tid in v[i], so the first 4 and 8 items are
// the 512 x 4 and 512 x 8 layouts of the row's first 2048 and 4096 keys),
// and the row is selected whole from registers in the smallest of those
// shapes that holds it, without a second round trip for its scores.
constexpr int kMidMaxColumns = 8192;

template <int K, int N>
__device__ __forceinline__ void take_items(const uint32_t (&v)[N], const int (&pg)[N],
                                           uint32_t (&vk)[K], int (&pk)[K]) {
#pragma unroll
  for (int i = 0; i < K; ++i) {
    vk[i] = v[i];
    pk[i] = pg[i];
  }
}

template <int D, int NKV, int WAVES, int ITEMS, int WIDE>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(2)))
void select_attend_kernel(const FusedSelect a, const AttnParams p) {
  constexpr int kThreads = 64 * WAVES;
  using Lds = AttnLds<D, NKV, WAVES, true>;
  using Topk = FusedTopkLds<kThreads, ITEMS>;
  constexpr int kSelBytes =
      WIDE && (int)sizeof(FusedWideLds) > (int)sizeof(Topk) ? (int)sizeof(FusedWideLds)
                                                             : (int)sizeof(Topk);
  constexpr int kBytes = Lds::kBufBytes > kSelBytes ? Lds::kBufBytes : kSelBytes;
  __shared__ __attribute__((aligned(16))) char s_lds[kBytes];
  __shared__ float s_m[WAVES][16];
  __shared__ float s_l[WAVES][16];
  __shared__ __attribute__((aligned(16))) int s_idx[kFusedMaxWidth];
  auto& tk = *reinterpret_cast<Topk*>(s_lds);
  const int row = blockIdx.x;
  const float* srow = a.scores + (int64_t)row * a.score_row_stride;
  RowMeta r;
  if constexpr (WIDE == 2) {
    static_assert(kThreads == kWideThreads && ITEMS == 4, "the 512 x 4 shape of 2048 columns");
    constexpr int kMidItems = kMidMaxColumns / kThreads;
    const DirectLoader load{srow, 0};
    uint32_t v[kMidItems];
    int pg[kMidItems];
    load_scores<kThreads, kMidItems>(load, a.cols, v);
    const RowRequest q =
        load_request<kThreads, kMidItems, true, true>(load, a.cols, a.meta, row, pg);
    // Nothing below may wait for the length before the loads above are out.
    __builtin_amdgcn_sched_barrier(0);
    const int length = a.lengths[row];
    const int whole = max(min(max(length, 0), a.cols), 2 * a.topk);
    auto& wide = *reinterpret_cast<FusedWideLds*>(s_lds);
#define QSA_MID_ROW(K, LIMIT)                                                                  \
  {                                                                                            \
    using Stage = TopkStage<kThreads, K, true>;                                                \
    auto& st = *reinterpret_cast<Stage*>(wide.stage);                                          \
    uint32_t vk[K];                                                                            \
    int pk[K];                                                                                 \
    take_items<K>(v, pg, vk, pk);                                                              \
    r = process_loaded_whole<kThreads, K, true, true, true>(                                   \
        load, LIMIT, vk, pk,                                                                   \
        [&] { return load_pages<kThreads, K, true, true>(load, LIMIT, a.meta, q, pk); },       \
        length, a.cols, a.topk, a.meta, row, s_idx, wide.sh, st, reinterpret_cast<int*>(st.key)); \
  }
    if (whole <= kThreads * 4) QSA_MID_ROW(4, kThreads * 4)
    else if (whole <= kThreads * 8) QSA_MID_ROW(8, kThreads * 8)
    else QSA_MID_ROW(kMidItems, a.cols)
#undef QSA_MID_ROW
  } else if constexpr (WIDE == 1) {
    static_assert(kThreads == kWideThreads && ITEMS == 4, "the 512 x 4 shape of 2048 columns");
    constexpr int kNarrowCols = kThreads * ITEMS;
    const DirectLoader load{srow, 0};
    uint32_t v[ITEMS];
    int pg[ITEMS];
    load_scores<kThreads, ITEMS>(load, kNarrowCols, v);
    const RowRequest q =
        load_request<kThreads, ITEMS, true, true>(load, kNarrowCols, a.meta, row, pg);
    // Nothing below may wait for the length before the loads above are out.
    __builtin_amdgcn_sched_barrier(0);
    const int length = a.lengths[row];
    // Rows longer than 2048 keys are rare in a wide class: the hint keeps
    // the long-row selection's code out of the way of the common path, which
    // with it runs straight into the attention (measured: the serving width's
    // step 42.4 -> 41.2 us and decode_long_skew's 25.4 -> 24.4 us, with the
    // same instructions otherwise).
    if (__builtin_expect(min(length, a.cols) <= kNarrowCols, 1)) {  // uniform
      r = process_loaded_whole<kThreads, ITEMS, true, true, true>(
          load, kNarrowCols, v, pg,
          [&] { return load_pages<kThreads, ITEMS, true, true>(load, kNarrowCols, a.meta, q, pg); },
          length, a.cols, a.topk, a.meta, row, s_idx, tk.sh, tk.st,
          reinterpret_cast<int*>(tk.st.key));
    } else {
      auto& wide = *reinterpret_cast<FusedWideLds*>(s_lds);
      r = select_wide_row(srow, a.cols, length, a.topk, a.meta, row, s_idx, wide.sh, wide.stage);
    }
  } else {
    r = process_row_whole<kThreads, ITEMS, true, true, decltype(tk.st), true>(
        DirectLoader{srow, 0}, a.cols, a.lengths[row], a.cols, a.topk, a.meta, row, s_idx, tk.sh,
        tk.st, reinterpret_cast<int*>(tk.st.key));
  }
  const int count = expanded_span(a.meta, r, a.topk).count(r);
  __syncthreads();  // the row is in s_idx; the top-k's LDS is free for the attention
  attend<D, NKV, WAVES, true, true, true>(p, row, blockIdx.y, blockIdx.z, s_idx, count, s_lds,
                                          s_m, s_l);
  if (blockIdx.y == 0 && blockIdx.z == 0) {
    int32_t* irow = a.indices + (int64_t)row * a.indices_row_stride;
    for (int c = threadIdx.x; c < a.meta.out_width; c += kThreads) irow[c] = s_idx[c];
    if (threadIdx.x == 0) a.counts[row] = count;
  }
}

// LSE merge of split partials (ops/qsa.py:306-362). One thread per (row, head,
// 4 dims); a thread issues the loads of up to kMergeChunk splits at once so a
// merge costs one memory round trip per chunk. The grid is (rows, parts of a
// row): workgroups are dispatched round-robin over the XCDs in linear order,
// so with a row count that is a multiple of 8 every workgroup of row r runs on
// XCD r mod 8, the XCD whose attention workgroups (grid (rows, splits, head
// groups)) wrote that row's partials, and the partials are read from that
// XCD's L2 instead of from another's write-back.
__global__ __launch_bounds__(256) void merge_kernel(const float* __restrict__ part_out,
                                                    const float* __restrict__ part_lse,
                                                    int num_splits, int rows, int num_q_heads,
                                                    int head_dim, uint16_t* out, int64_t out_row,
                                                    int64_t out_head, const uint16_t* gate,
                                                    int64_t g_row, int64_t g_head, int64_t g_dim) {
  const int chunks = head_dim / 4;
  const int item = (int)blockIdx.y * (int)blockDim.x + (int)threadIdx.x;  // within the row
  if (item >= num_q_heads * chunks) return;
  const int row = blockIdx.x;
  const int head = item / chunks;
  const int d0 = (item % chunks) * 4;
  const int64_t rh = (int64_t)row * num_q_heads + head;
  const int64_t split_stride = (int64_t)rows * num_q_heads;
  float lmax = -INFINITY, den = 0.0f;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < num_splits; s0 += kMergeChunk) {
    float lse[kMergeChunk];
    float4 v[kMergeChunk];
#pragma unroll
    for (int c = 0; c < kMergeChunk; ++c) {
      const int64_t pr = (int64_t)(s0 + c) * split_stride + rh;
      const bool ok = s0 + c < num_splits;
      lse[c] = ok ? part_lse[pr] : -INFINITY;
      v[c] = ok ? *reinterpret_cast<const float4*>(part_out + pr * head_dim + d0)
                : float4{0.f, 0.f, 0.f, 0.f};
    }
    float cmax = lmax;
#pragma unroll
    for (int c = 0; c < kMergeChunk; ++c) cmax = fmaxf(cmax, lse[c]);
    if (cmax == -INFINITY) continue;
    const float rescale = fast_exp2(lmax - cmax);  // 0 while nothing has been merged
    den *= rescale;
    for (int d = 0; d < 4; ++d) acc[d] *= rescale;
#pragma unroll
    for (int c = 0; c < kMergeChunk; ++c) {
      const float w = fast_exp2(lse[c] - cmax);
      den += w;
      acc[0] += w * v[c].x;
      acc[1] += w * v[c].y;
      acc[2] += w * v[c].z;
      acc[3] += w * v[c].w;
    }
    lmax = cmax;
  }
  float o[4];
  for (int d = 0; d < 4; ++d) o[d] = den > 0.0f ? acc[d] / den : 0.0f;
  uint16_t* optr = out + (int64_t)row * out_row + (int64_t)head * out_head + d0;
  if (gate) {
    const uint16_t* gptr = gate + (int64_t)row * g_row + (int64_t)head * g_head;
    for (int d = 0; d < 4; d += 2) {
      const uint32_t ob = pack_bf16x2(o[d], o[d + 1]);
      o[d] = bf16_lo(ob) * sigmoidf_(bf16_lo((uint32_t)gptr[(int64_t)(d0 + d) * g_dim]));
      o[d + 1] = bf16_hi(ob) * sigmoidf_(bf16_lo((uint32_t)gptr[(int64_t)(d0 + d + 1) * g_dim]));
    }
  }
  *reinterpret_cast<uint32_t*>(optr) = pack_bf16x2(o[0], o[1]);
  *reinterpret_cast<uint32_t*>(optr + 2) = pack_bf16x2(o[2], o[3]);
}

struct HeadPlan {
  int nkv;             // kv heads per head group
  int heads_per_wave;  // query-head slots used (<= 16)
  int groups;          // head groups per row
};

// Decode (physical) rows stream their K/V from HBM. Measured on MI355X (16 q /
// 2 kv heads x 128, top-k 2048 tokens, four rotating query sets so the
// selected K/V is not served by the Infinity Cache): a full round of 8-wave
// workgroups (one per CU) streams fastest, and one kv head per workgroup is
// the cheapest way to reach it (batch 128: 256 workgroups without a split 49.7
// us, against 53.2 us for both kv heads per workgroup in 2 splits plus the
// merge; batch 16: 8 splits 12.0 us against 16.2 us). A split pays for its
// merge below ~160 workgroups (batch 64: 2 splits 27.5 us, none 29.4 us;
// batch 96: none 38.0 us, 2 splits 43.8 us). So physical rows group kv heads
// only while a full round remains, and split smaller batches up to a round but
// never past it: a second, partial round of workgroups costs about as much as
// the first (batch 48: 2 splits 22.9 us, 4 splits 24.6; batch 36: 2 splits
// 18.7, 4 splits 22.7; batch 24: 4 splits 14.2, 8 splits 15.0; contexts
// U[8192, 32768], four query sets with their own selections). Nor below 8
// tiles (256 tokens) per split: shorter splits add partials to merge faster
// than they shorten the launch (batch 8 of 2055 tokens: 4 splits 11.9 us, 8
// splits 10.3, 16 splits 10.9, 32 splits 12.7, merge included).
constexpr int kDecodeRoundWorkgroups = 256;
constexpr int kDecodeNoSplitWorkgroups = 160;
constexpr int kDecodeMinSplitTiles = 8;

bool plan_heads(int num_q_heads, int num_kv_heads, int rows, bool physical, HeadPlan* plan) {
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads) return false;
  const int group = num_q_heads / num_kv_heads;
  if (group > 16) {
    if (group % 16) return false;
    plan->nkv = 1;
    plan->heads_per_wave = 16;
  } else {
    int nkv = 1;
    for (int cand : {4, 2, 1}) {
      if (cand * group <= 16 && num_kv_heads % cand == 0) {
        nkv = cand;
        break;
      }
    }
    if (physical)
      while (nkv > 1 && (int64_t)rows * (num_q_heads / (nkv * group)) < kDecodeRoundWorkgroups)
        nkv /= 2;
    plan->nkv = nkv;
    plan->heads_per_wave = nkv * group;
  }
  plan->groups = num_q_heads / plan->heads_per_wave;
  return true;
}

// Waves per workgroup. Physical (decode) rows take 8 at every batch: on the
// 64-row, 16-head decode shape 8 waves x 4 splits measured faster than 4 waves
// x 8 splits, and small batches (1 to 31 rows, four rotating query sets) ran
// the attention alone 0.0-0.4 us faster with 8 waves than with 4 and, through
// the combined selection + attention launch that 8 waves make possible,
// 1.5-2 us faster than as two launches. Logical (prefill) rows always take 4 waves: at 256
// registers a lane two such workgroups share a CU, so one row's start (index ->
// table -> K round trips) overlaps the other's streaming; measured 5.11 ms
// against 5.58 ms with 8 waves on the 32768-row chunked prefill. D = 128 with
// 4 kv heads per group needs more than the 256 registers a lane gets at two
// waves per SIMD, so it always runs 4 waves (one per SIMD).
bool fits_8_waves(int head_dim, int nkv) { return !(head_dim == 128 && nkv == 4); }
int waves_for(const HeadPlan& plan, int head_dim, bool physical) {
  if (!physical) return 4;
  return fits_8_waves(head_dim, plan.nkv) ? 8 : 4;
}

template <int D, int NKV, bool PHYSICAL, bool BUF>
hipError_t launch_attn_mode(const AttnParams& p, dim3 grid, int waves, hipStream_t stream) {
  if constexpr (PHYSICAL && !(D == 128 && NKV == 4)) {
    if (waves == 8) {
      hipLaunchKernelGGL((sparse_attn_kernel<D, NKV, 8, PHYSICAL, BUF>), grid, dim3(512), 0, stream,
                         p);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((sparse_attn_kernel<D, NKV, 4, PHYSICAL, BUF>), grid, dim3(256), 0, stream, p);
  return hipGetLastError();
}

// Physical and logical indices are separate kernels: the logical form's
// block-table loads would otherwise make every wait in the loop conservative.
// Logical rows always run 4 waves (waves_for).
// Buffer addressing serves physical (decode) rows only: on the 32768-row
// chunked prefill the logical kernel measured ~2% slower with it (5.24 against
// 5.12 ms), decode ~2% faster (26.7 against 27.2 us at batch 64).
template <int D, int NKV>
hipError_t launch_attn(const AttnParams& p, dim3 grid, int waves, bool buf, hipStream_t stream) {
  if (!p.physical) return launch_attn_mode<D, NKV, false, false>(p, grid, waves, stream);
  return buf ? launch_attn_mode<D, NKV, true, true>(p, grid, waves, stream)
             : launch_attn_mode<D, NKV, true, false>(p, grid, waves, stream);
}

// Whether the K/V views can be addressed through buffer resources: token-major
// (block stride = page_size x token stride), non-negative strides, and each kv
// head's rows within one 32-bit byte range.
bool buffer_addressable(int64_t kb, int64_t kt, int64_t kh, int64_t vb, int64_t vt, int64_t vh,
                        int page_size, int num_slots, int num_kv_heads, int head_dim,
                        uint32_t* k_bytes, uint32_t* v_bytes) {
  if (kt <= 0 || vt <= 0 || kh < 0 || vh < 0) return false;
  if (kb != (int64_t)page_size * kt || vb != (int64_t)page_size * vt) return false;
  const int64_t row = (int64_t)head_dim * 2;
  const int64_t kr = num_slots > 0 ? (int64_t)(num_slots - 1) * kt + row : 0;
  const int64_t vr = num_slots > 0 ? (int64_t)(num_slots - 1) * vt + row : 0;
  const int64_t kho = (int64_t)(num_kv_heads - 1) * kh, vho = (int64_t)(num_kv_heads - 1) * vh;
  if (kr > kMaxBufferBytes || vr > kMaxBufferBytes || kho > INT32_MAX || vho > INT32_MAX)
    return false;
  *k_bytes = (uint32_t)kr;
  *v_bytes = (uint32_t)vr;
  return true;
}

int launch_merge(const float* part_out, const float* part_lse, int num_splits, int rows,
                 int num_q_heads, int head_dim, uint16_t* out, int64_t out_row, int64_t out_head,
                 const uint16_t* gate, int64_t g_row, int64_t g_head, int64_t g_dim,
                 hipStream_t s) {
  const int64_t parts = ((int64_t)num_q_heads * (head_dim / 4) + 255) / 256;
  if (parts > 65535) return fail(QSA_ERR_UNSUPPORTED, "qsa_sparse_attention merge: too many heads");
  const dim3 grid((unsigned)rows, (unsigned)parts);
  hipLaunchKernelGGL(merge_kernel, grid, dim3(256), 0, s, part_out, part_lse, num_splits, rows,
                     num_q_heads, head_dim, out, out_row, out_head, gate, g_row, g_head, g_dim);
  return check_launch("qsa_sparse_attention merge launch");
}

}  // namespace
}  // namespace qsa

#ifdef QSA_ATTN_WIDE_UNIT

namespace qsa {
namespace {
template <int D, int NKV>
void launch_wide(bool mid, dim3 grid, const FusedSelect& a, const AttnParams& p,
                 hipStream_t stream) {
  if (mid)
    hipLaunchKernelGGL((select_attend_kernel<D, NKV, 8, 4, 2>), grid, dim3(512), 0, stream, a, p);
  else
    hipLaunchKernelGGL((select_attend_kernel<D, NKV, 8, 4, 1>), grid, dim3(512), 0, stream, a, p);
}
}  // namespace
}  // namespace qsa

extern "C" __attribute__((visibility("hidden"))) int qsa_attn_launch_fused_wide(
    const void* select, size_t select_bytes, const void* params, size_t params_bytes,
    unsigned grid_x, unsigned grid_y, unsigned grid_z, int head_dim, int nkv, hipStream_t stream) {
  using namespace qsa;
  if (select_bytes != sizeof(FusedSelect) || params_bytes != sizeof(AttnParams))
    return (int)hipErrorInvalidValue;
  FusedSelect a;
  AttnParams p;
  std::memcpy(&a, select, sizeof a);
  std::memcpy(&p, params, sizeof p);
  const dim3 grid(grid_x, grid_y, grid_z);
  const bool mid = a.cols <= kMidMaxColumns;
  if (head_dim == 128 && nkv == 1)
    launch_wide<128, 1>(mid, grid, a, p, stream);
  else if (head_dim == 128)
    launch_wide<128, 2>(mid, grid, a, p, stream);
  else if (nkv == 1)
    launch_wide<64, 1>(mid, grid, a, p, stream);
  else
    launch_wide<64, 2>(mid, grid, a, p, stream);
  return (int)hipGetLastError();
}

#else  // the library's entry points

using namespace qsa;

extern "C" int qsa_sparse_attention_splits(int rows, int num_q_heads, int num_kv_heads,
                                           int head_dim, int width, int use_decode_kernel) {
  HeadPlan plan;
  const bool physical = use_decode_kernel != 0;
  if (rows <= 0 || !plan_heads(num_q_heads, num_kv_heads, rows, physical, &plan)) return 1;
  const int tiles = (width + kTile - 1) / kTile;
  const int64_t base = (int64_t)rows * plan.groups;
  // At least two tiles per split (a one-tile split pays for a partial and its
  // merge for nothing). The decode kernel takes physical slots (splits as
  // measured, above) and keeps at least kDecodeMinSplitTiles tiles per split;
  // prefill rows (logical ids, 4-wave workgroups, two per CU) split up to two
  // workgroups per CU.
  int splits = 1;
  if (physical) {
    if (base < kDecodeNoSplitWorkgroups)
      while (splits * 2 * base <= kDecodeRoundWorkgroups &&
             splits * 2 <= std::max(1, tiles / kDecodeMinSplitTiles) && splits < 64)
        splits *= 2;
  } else {
    const int64_t target = 2 * kCUs;
    while (splits * 2 * base <= target && splits * 2 <= std::max(1, tiles / 2) && splits < 64)
      splits *= 2;
  }
  return splits;
}

extern "C" size_t qsa_sparse_attention_workspace_bytes(int rows, int num_q_heads, int head_dim,
                                                       int num_splits) {
  if (num_splits <= 1 || rows <= 0) return 0;
  const size_t n = (size_t)num_splits * rows * num_q_heads;
  return n * head_dim * sizeof(float) + n * sizeof(float);
}

namespace qsa {
namespace {

// A validated attention call: its parameters and launch plan.
struct AttnLaunch {
  AttnParams p;
  HeadPlan plan;
  dim3 grid;
  int waves;
  bool buf;
  int head_dim;
  int64_t out_row, out_head, g_row, g_head, g_dim;
};

// Checks qsa_sparse_attention's arguments (rows > 0) and fills the launch.
int prepare_attention(
    const void* q, int64_t q_row_stride, int64_t q_head_stride, int rows, int num_q_heads,
    int head_dim, const void* k_cache, int64_t k_block_stride, int64_t k_token_stride,
    int64_t k_head_stride, const void* v_cache, int64_t v_block_stride, int64_t v_token_stride,
    int64_t v_head_stride, int num_blocks, int page_size, int num_kv_heads,
    const int32_t* indices, int64_t indices_row_stride, int width, const int32_t* block_table,
    int64_t table_row_stride, int table_width, int num_requests, const int32_t* token_to_req,
    const int32_t* valid_counts, void* out, int64_t out_row_stride, int64_t out_head_stride,
    const void* gate, int64_t gate_row_stride, int64_t gate_head_stride, int64_t gate_dim_stride,
    int indices_are_physical, int num_splits, void* workspace, size_t workspace_bytes,
    AttnLaunch* L) {
  if (head_dim != 64 && head_dim != 128)
    return fail(QSA_ERR_UNSUPPORTED, "qsa_sparse_attention: head_dim must be 64 or 128");
  HeadPlan plan;
  if (!plan_heads(num_q_heads, num_kv_heads, rows, indices_are_physical != 0, &plan))
    return fail(QSA_ERR_UNSUPPORTED,
                "qsa_sparse_attention: query heads must be a multiple of kv heads with a GQA "
                "group that divides 16 or is a multiple of 16");
  if (!q || !k_cache || !v_cache || !indices || !token_to_req || !out)
    return fail(QSA_ERR_INVALID, "qsa_sparse_attention: null tensor pointer");
  if (!indices_are_physical && (!block_table || table_width <= 0 || num_requests <= 0))
    return fail(QSA_ERR_INVALID, "qsa_sparse_attention: logical indices need a block table");
  if (page_size <= 0 || num_blocks < 0 || width < 0)
    return fail(QSA_ERR_INVALID, "qsa_sparse_attention: bad page_size/num_blocks/width");
  if ((int64_t)num_blocks * page_size > INT32_MAX)
    return fail(QSA_ERR_UNSUPPORTED, "qsa_sparse_attention: more than 2^31 cache slots");
  if (num_splits < 1 || num_splits > 1024)
    return fail(QSA_ERR_INVALID, "qsa_sparse_attention: num_splits out of range");
  const size_t need = qsa_sparse_attention_workspace_bytes(rows, num_q_heads, head_dim, num_splits);
  if (need && (!workspace || workspace_bytes < need))
    return fail(QSA_ERR_WORKSPACE, "qsa_sparse_attention: workspace too small for split partials");
  if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) & 15u ||
      (q_row_stride | q_head_stride | k_block_stride | k_token_stride | k_head_stride |
       v_block_stride | v_token_stride | v_head_stride) & 7)
    return fail(QSA_ERR_INVALID,
                "qsa_sparse_attention: q/k/v must be 16-byte aligned with strides that are "
                "multiples of 8 elements");
  if (((uintptr_t)out & 3u) || (out_row_stride | out_head_stride) & 1)
    return fail(QSA_ERR_INVALID, "qsa_sparse_attention: out must be 4-byte aligned with even strides");
  if (need && ((uintptr_t)workspace & 15u))
    return fail(QSA_ERR_INVALID, "qsa_sparse_attention: workspace must be 16-byte aligned");

  AttnParams p;
  p.q = static_cast<const uint16_t*>(q);
  p.q_row = q_row_stride;
  p.q_head = q_head_stride;
  p.k = static_cast<const char*>(k_cache);
  p.v = static_cast<const char*>(v_cache);
  p.kb = k_block_stride * 2;
  p.kt = k_token_stride * 2;
  p.kh = k_head_stride * 2;
  p.vb = v_block_stride * 2;
  p.vt = v_token_stride * 2;
  p.vh = v_head_stride * 2;
  p.num_blocks = num_blocks;
  p.page_size = page_size;
  p.page_div = FastDiv::make(page_size);
  p.indices = indices;
  p.idx_row = indices_row_stride;
  p.width = width;
  p.table = block_table ? block_table : indices;
  p.table_row = table_row_stride;
  p.table_width = table_width;
  p.num_requests = num_requests;
  p.token_to_req = token_to_req;
  p.valid_counts = valid_counts;
  p.out = static_cast<uint16_t*>(out);
  p.out_row = out_row_stride;
  p.out_head = out_head_stride;
  p.gate = static_cast<const uint16_t*>(gate);
  p.g_row = gate_row_stride;
  p.g_head = gate_head_stride;
  p.g_dim = gate_dim_stride;
  const size_t n_part = (size_t)num_splits * rows * num_q_heads;
  p.part_out = need ? static_cast<float*>(workspace) : nullptr;
  p.part_lse = need ? static_cast<float*>(workspace) + n_part * head_dim : nullptr;
  p.rows = rows;
  p.num_q_heads = num_q_heads;
  p.group = num_q_heads / num_kv_heads;
  p.heads_per_wave = plan.heads_per_wave;
  p.num_splits = num_splits;
  p.physical = indices_are_physical ? 1 : 0;
  p.scale_log2 = (float)(1.0 / __builtin_sqrt((double)head_dim) * 1.4426950408889634);

  if (plan.groups > 65535 || num_splits > 65535)
    return fail(QSA_ERR_UNSUPPORTED, "qsa_sparse_attention: grid too large");
  p.num_slots = num_blocks * page_size;
  p.k_bytes = p.v_bytes = 0;
  L->buf = buffer_addressable(p.kb, p.kt, p.kh, p.vb, p.vt, p.vh, page_size, p.num_slots,
                              num_kv_heads, head_dim, &p.k_bytes, &p.v_bytes);
  p.kt32 = L->buf ? (uint32_t)p.kt : 0;
  p.vt32 = L->buf ? (uint32_t)p.vt : 0;
  L->p = p;
  L->plan = plan;
  L->grid = dim3(rows, num_splits, plan.groups);
  L->waves = waves_for(plan, head_dim, indices_are_physical != 0);
  L->head_dim = head_dim;
  L->out_row = out_row_stride;
  L->out_head = out_head_stride;
  L->g_row = gate_row_stride;
  L->g_head = gate_head_stride;
  L->g_dim = gate_dim_stride;
  return QSA_OK;
}

// The merge of a launch's split partials (none with one split).
int merge_splits(const AttnLaunch& L, hipStream_t s) {
  const AttnParams& p = L.p;
  if (p.num_splits <= 1) return QSA_OK;
  return launch_merge(p.part_out, p.part_lse, p.num_splits, p.rows, p.num_q_heads, L.head_dim,
                      p.out, L.out_row, L.out_head, p.gate, L.g_row, L.g_head, L.g_dim, s);
}

int launch_attention(const AttnLaunch& L, hipStream_t s) {
  const AttnParams& p = L.p;
  hipError_t err = hipSuccess;
  if (L.head_dim == 128) {
    if (L.plan.nkv == 1) err = launch_attn<128, 1>(p, L.grid, L.waves, L.buf, s);
    else if (L.plan.nkv == 2) err = launch_attn<128, 2>(p, L.grid, L.waves, L.buf, s);
    else err = launch_attn<128, 4>(p, L.grid, L.waves, L.buf, s);
  } else {
    if (L.plan.nkv == 1) err = launch_attn<64, 1>(p, L.grid, L.waves, L.buf, s);
    else if (L.plan.nkv == 2) err = launch_attn<64, 2>(p, L.grid, L.waves, L.buf, s);
    else err = launch_attn<64, 4>(p, L.grid, L.waves, L.buf, s);
  }
  if (err != hipSuccess)
    return fail(QSA_ERR_HIP, std::string("qsa_sparse_attention launch: ") + hipGetErrorString(err));
  return merge_splits(L, s);
}

}  // namespace
}  // namespace qsa

extern "C" int qsa_sparse_attention(
    const void* q, int64_t q_row_stride, int64_t q_head_stride, int rows, int num_q_heads,
    int head_dim, const void* k_cache, int64_t k_block_stride, int64_t k_token_stride,
    int64_t k_head_stride, const void* v_cache, int64_t v_block_stride, int64_t v_token_stride,
    int64_t v_head_stride, int num_blocks, int page_size, int num_kv_heads,
    const int32_t* indices, int64_t indices_row_stride, int width, const int32_t* block_table,
    int64_t table_row_stride, int table_width, int num_requests, const int32_t* token_to_req,
    const int32_t* valid_counts, void* out, int64_t out_row_stride, int64_t out_head_stride,
    const void* gate, int64_t gate_row_stride, int64_t gate_head_stride, int64_t gate_dim_stride,
    int indices_are_physical, int num_splits, void* workspace, size_t workspace_bytes,
    void* stream) {
  if (rows < 0) return fail(QSA_ERR_INVALID, "qsa_sparse_attention: rows < 0");
  if (rows == 0) return QSA_OK;
  AttnLaunch L;
  const int st = prepare_attention(
      q, q_row_stride, q_head_stride, rows, num_q_heads, head_dim, k_cache, k_block_stride,
      k_token_stride, k_head_stride, v_cache, v_block_stride, v_token_stride, v_head_stride,
      num_blocks, page_size, num_kv_heads, indices, indices_row_stride, width, block_table,
      table_row_stride, table_width, num_requests, token_to_req, valid_counts, out,
      out_row_stride, out_head_stride, gate, gate_row_stride, gate_head_stride, gate_dim_stride,
      indices_are_physical, num_splits, workspace, workspace_bytes, &L);
  if (st != QSA_OK) return st;
  return launch_attention(L, static_cast<hipStream_t>(stream));
}

namespace qsa {
namespace {

// Rows below which the top-k runs one workgroup per row for rows of up to
// 2048 columns (its latency-bound launch shapes), the shapes the fused kernel
// reuses.
constexpr int kFusedMaxRows = 1024;
constexpr int kFusedMaxColumns = 2048;

// Keys per thread of the fused selection (512 threads): every row of up to
// `cols` keys in the workgroup's registers; a wider buffer starts with its
// rows' first 2048 columns (the WIDE kernel).
int fused_items(int cols) { return cols <= 1024 ? 2 : 4; }

// Whether a decode batch's selection and attention run as one launch: the
// top-k's 512-thread shapes (rows < 1024, at most kWideMaxColumns columns, the
// selected ids within the key stage), an expanded row that fits LDS, and the
// attention's 8-wave, buffer-addressed plan with at most 2 kv heads per
// workgroup. 4-wave workgroups (D = 128 with 4 kv heads per group) keep two
// launches: a 256-thread selection inside them cost as much as the launch it
// removed (batch 1, 4, 8, 16, 24, 31 of decode_32k's shapes when those batches
// ran 4 waves: 17.93 / 18.76 / 19.66 / 22.57 / 26.09 / 28.44 us as two
// launches, 17.96 / 19.19 / 19.94 / 22.67 / 26.04 / 28.52 combined).
bool fuses(int rows, int cols, int width, int ratio, int waves, bool buf, int nkv) {
  const int topk = ratio > 0 ? width / ratio : 0;
  return rows > 0 && rows < kFusedMaxRows && cols <= kWideMaxColumns && topk > 0 &&
         2 * topk <= 512 * fused_items(cols) && width <= kFusedMaxWidth && waves == 8 && buf &&
         nkv <= 2;
}

template <int D, int NKV>
hipError_t launch_fused(const FusedSelect& a, const AttnLaunch& L, hipStream_t s) {
  if (a.cols > kFusedMaxColumns)
    return (hipError_t)qsa_attn_launch_fused_wide(&a, sizeof a, &L.p, sizeof L.p, L.grid.x,
                                                  L.grid.y, L.grid.z, D, NKV, s);
  if (fused_items(a.cols) == 2)
    hipLaunchKernelGGL((select_attend_kernel<D, NKV, 8, 2, 0>), L.grid, dim3(512), 0, s, a,
                       L.p);
  else
    hipLaunchKernelGGL((select_attend_kernel<D, NKV, 8, 4, 0>), L.grid, dim3(512), 0, s, a,
                       L.p);
  return hipGetLastError();
}

}  // namespace
}  // namespace qsa

extern "C" int qsa_decode_select_attention_fuses(int rows, int cols, int width, int ratio,
                                                 int num_q_heads, int num_kv_heads,
                                                 int head_dim) {
  HeadPlan plan;
  if ((head_dim != 64 && head_dim != 128) || !plan_heads(num_q_heads, num_kv_heads, rows, true, &plan))
    return 0;
  return fuses(rows, cols, width, ratio, waves_for(plan, head_dim, true), true, plan.nkv);
}

extern "C" size_t qsa_decode_select_attention_workspace_bytes(int rows, int cols, int width,
                                                              int ratio, int num_q_heads,
                                                              int head_dim, int num_splits) {
  if (rows <= 0 || ratio <= 0) return 0;
  const size_t sel = qsa_topk_workspace_bytes(rows, cols, width / ratio);
  const size_t att = qsa_sparse_attention_workspace_bytes(rows, num_q_heads, head_dim, num_splits);
  return std::max(sel, att);
}

extern "C" int qsa_decode_select_attention(
    const float* scores, int64_t score_row_stride, int rows, int cols, const int32_t* lengths,
    const int64_t* positions, const int32_t* sequence_lengths, int num_requests,
    const int32_t* token_to_req, const int32_t* block_table, int64_t table_row_stride,
    int table_width, int ratio, int32_t* indices, int64_t indices_row_stride, int width,
    int32_t* counts, const void* q, int64_t q_row_stride, int64_t q_head_stride, int num_q_heads,
    int head_dim, const void* k_cache, int64_t k_block_stride, int64_t k_token_stride,
    int64_t k_head_stride, const void* v_cache, int64_t v_block_stride, int64_t v_token_stride,
    int64_t v_head_stride, int num_blocks, int page_size, int num_kv_heads, void* out,
    int64_t out_row_stride, int64_t out_head_stride, const void* gate, int64_t gate_row_stride,
    int64_t gate_head_stride, int64_t gate_dim_stride, int num_splits, void* workspace,
    size_t workspace_bytes, void* stream) {
  const char* name = "qsa_decode_select_attention";
  if (rows < 0 || cols < 0) return fail(QSA_ERR_INVALID, std::string(name) + ": negative shape");
  if (rows == 0) return QSA_OK;
  if (ratio <= 0) return fail(QSA_ERR_INVALID, std::string(name) + ": ratio must be positive");
  const int topk = width / ratio;
  if (topk <= 0) return fail(QSA_ERR_INVALID, std::string(name) + ": topk must be positive");
  if (!scores || !lengths || !indices || !counts || !positions || !sequence_lengths ||
      !token_to_req || !block_table)
    return fail(QSA_ERR_INVALID, std::string(name) + ": null selection pointer");
  if (num_splits <= 0)
    num_splits = qsa_sparse_attention_splits(rows, num_q_heads, num_kv_heads, head_dim, width, 1);
  AttnLaunch L;
  int st = prepare_attention(
      q, q_row_stride, q_head_stride, rows, num_q_heads, head_dim, k_cache, k_block_stride,
      k_token_stride, k_head_stride, v_cache, v_block_stride, v_token_stride, v_head_stride,
      num_blocks, page_size, num_kv_heads, indices, indices_row_stride, width, block_table,
      table_row_stride, table_width, num_requests, token_to_req, counts, out, out_row_stride,
      out_head_stride, gate, gate_row_stride, gate_head_stride, gate_dim_stride, 1, num_splits,
      workspace, workspace_bytes, &L);
  if (st != QSA_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!fuses(rows, cols, width, ratio, L.waves, L.buf, L.plan.nkv)) {
    st = qsa_topk_expand(scores, score_row_stride, rows, cols, lengths, positions,
                         sequence_lengths, num_requests, token_to_req, block_table,
                         table_row_stride, table_width, indices, indices_row_stride, 1, width,
                         counts, ratio, page_size, 1, 1, workspace, workspace_bytes, stream);
    if (st != QSA_OK) return st;
    return launch_attention(L, s);
  }
  FusedSelect a = {};
  a.scores = scores;
  a.score_row_stride = score_row_stride;
  a.lengths = lengths;
  a.cols = cols;
  a.topk = topk;
  a.meta = make_expand_meta(positions, sequence_lengths, num_requests, token_to_req, block_table,
                            table_row_stride, table_width, nullptr, 1, width, ratio, page_size,
                            1, 0);
  a.indices = indices;
  a.indices_row_stride = indices_row_stride;
  a.counts = counts;
  hipError_t err;
  if (head_dim == 128)
    err = L.plan.nkv == 1 ? launch_fused<128, 1>(a, L, s) : launch_fused<128, 2>(a, L, s);
  else
    err = L.plan.nkv == 1 ? launch_fused<64, 1>(a, L, s) : launch_fused<64, 2>(a, L, s);
  if (err != hipSuccess)
    return fail(QSA_ERR_HIP, std::string(name) + " launch: " + hipGetErrorString(err));
  return merge_splits(L, s);
}

extern "C" int qsa_sparse_attention_merge(const float* partial_out, const float* partial_lse,
                                          int num_splits, int rows, int num_q_heads, int head_dim,
                                          void* out, int64_t out_row_stride,
                                          int64_t out_head_stride, const void* gate,
                                          int64_t gate_row_stride, int64_t gate_head_stride,
                                          int64_t gate_dim_stride, void* stream) {
  if (rows < 0 || num_splits < 1 || num_q_heads <= 0 || head_dim <= 0 || head_dim % 4)
    return fail(QSA_ERR_INVALID, "qsa_sparse_attention_merge: bad shape");
  if (rows == 0) return QSA_OK;
  if (!partial_out || !partial_lse || !out)
    return fail(QSA_ERR_INVALID, "qsa_sparse_attention_merge: null tensor pointer");
  if (((uintptr_t)partial_out & 15u) || ((uintptr_t)out & 3u) || (out_row_stride | out_head_stride) & 1)
    return fail(QSA_ERR_INVALID, "qsa_sparse_attention_merge: misaligned partials or output");
  return launch_merge(partial_out, partial_lse, num_splits, rows, num_q_heads, head_dim,
                      static_cast<uint16_t*>(out), out_row_stride, out_head_stride,
                      static_cast<const uint16_t*>(gate), gate_row_stride, gate_head_stride,
                      gate_dim_stride, static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------
// qsa_sparse_attention_noalloc: qsa_sparse_attention with the split partials
// in `scratch`, a file-scope device array (each GPU the library runs on holds
// its own copy until the process ends), for callers that cannot allocate.
// Host code never passes `scratch` itself to a kernel (on the host its name
// is a stand-in, not a device address): the address of this GPU's copy comes
// from hipGetSymbolAddress, once per device, and is kept per device.
// ---------------------------------------------------------------------------
static __device__ __align__(256) float scratch[QSA_SPARSE_ATTENTION_SCRATCH_BYTES / sizeof(float)];

namespace {
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kScratchDevices] = {};

// This GPU's copy of `scratch`. The stream must belong to the current device
// (the one whose copy the address names).
int scratch_address(hipStream_t stream, void** out) {
  int current = -1;
  hipError_t err = hipGetDevice(&current);
  if (err != hipSuccess)
    return fail(QSA_ERR_HIP, std::string("qsa_sparse_attention_noalloc: hipGetDevice: ") +
                                 hipGetErrorString(err));
  if (stream) {
    hipDevice_t owner = -1;
    err = hipStreamGetDevice(stream, &owner);
    if (err != hipSuccess)
      return fail(QSA_ERR_HIP, std::string("qsa_sparse_attention_noalloc: hipStreamGetDevice: ") +
                                   hipGetErrorString(err));
    if (owner != current)
      return fail(QSA_ERR_INVALID,
                  "qsa_sparse_attention_noalloc: the stream belongs to device " +
                      std::to_string(owner) + " but device " + std::to_string(current) +
                      " is current");
  }
  if (current < 0 || current >= kScratchDevices)
    return fail(QSA_ERR_UNSUPPORTED, "qsa_sparse_attention_noalloc: device ordinal beyond 63");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[current]) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !ptr)
      return fail(QSA_ERR_HIP, std::string("qsa_sparse_attention_noalloc: hipGetSymbolAddress: ") +
                                   hipGetErrorString(err));
    g_scratch_ptr[current] = ptr;
  }
  *out = g_scratch_ptr[current];
  return QSA_OK;
}
}  // namespace

extern "C" int qsa_sparse_attention_noalloc(
    const void* q, int64_t q_row_stride, int64_t q_head_stride, int rows, int num_q_heads,
    int head_dim, const void* k_cache, int64_t k_block_stride, int64_t k_token_stride,
    int64_t k_head_stride, const void* v_cache, int64_t v_block_stride, int64_t v_token_stride,
    int64_t v_head_stride, int num_blocks, int page_size, int num_kv_heads,
    const int32_t* indices, int64_t indices_row_stride, int width, const int32_t* block_table,
    int64_t table_row_stride, int table_width, int num_requests, const int32_t* token_to_req,
    const int32_t* valid_counts, void* out, int64_t out_row_stride, int64_t out_head_stride,
    const void* gate, int64_t gate_row_stride, int64_t gate_head_stride, int64_t gate_dim_stride,
    int indices_are_physical, int num_splits, void* stream) {
  if (rows < 0 || num_q_heads < 0 || head_dim < 0)
    return fail(QSA_ERR_INVALID, "qsa_sparse_attention_noalloc: negative size");
  if (num_splits < 1 || num_splits > 1024)
    return fail(QSA_ERR_INVALID, "qsa_sparse_attention_noalloc: num_splits out of range");
  const size_t need = qsa_sparse_attention_workspace_bytes(rows, num_q_heads, head_dim, num_splits);
  if (need > QSA_SPARSE_ATTENTION_SCRATCH_BYTES)
    return fail(QSA_ERR_WORKSPACE,
                "qsa_sparse_attention_noalloc: split partials of " + std::to_string(need) +
                    " bytes exceed the " + std::to_string(QSA_SPARSE_ATTENTION_SCRATCH_BYTES) +
                    "-byte scratch (use fewer splits, or qsa_sparse_attention with a workspace)");
  // Every partial the merge reads is written by this call's attention launch,
  // so nothing in the scratch has to start at zero.
  void* partials = nullptr;
  if (need) {
    const int status = scratch_address(static_cast<hipStream_t>(stream), &partials);
    if (status != QSA_OK) return status;
  }
  return qsa_sparse_attention(
      q, q_row_stride, q_head_stride, rows, num_q_heads, head_dim, k_cache, k_block_stride,
      k_token_stride, k_head_stride, v_cache, v_block_stride, v_token_stride, v_head_stride,
      num_blocks, page_size, num_kv_heads, indices, indices_row_stride, width, block_table,
      table_row_stride, table_width, num_requests, token_to_req, valid_counts, out,
      out_row_stride, out_head_stride, gate, gate_row_stride, gate_head_stride, gate_dim_stride,
      indices_are_physical, num_splits, partials, need ? QSA_SPARSE_ATTENTION_SCRATCH_BYTES : 0,
      stream);
}

#endif  // QSA_ATTN_WIDE_UNIT
