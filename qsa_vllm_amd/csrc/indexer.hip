// Kernel 1: QSA indexer scoring, gfx950.
//
// logits[r, c] = D^-0.5 * sum_h relu(q[r, h, :] . K[c, :]) over the visible
// compressed keys of row r (ops/indexer.py:24-114 decode, :117-223 prefill),
// bf16 inputs, fp32 accumulation, written only for c < visible[r].
//
// Decode: a row's keys are only read once, so each wave streams key tiles of
// one row straight from HBM (GEMV-like, bandwidth bound), with the 16-key
// v_mfma_f32_16x16x32_bf16 layout of indexer_device.h: each load instruction
// reads 16 keys x 64 contiguous bytes.
//
// Prefill: consecutive query rows of a request see nearly the same keys, so an
// 8-wave workgroup owns 32 rows (4 per wave, their Q in registers) and stages
// each 64-key tile once in LDS, where all 32 rows reuse it (MFMA bound). It
// uses v_mfma_f32_32x32x16_bf16 with the index heads on M and 32 keys on N:
// A = Q[32 heads][16 dims] stays in registers, B = K^T[16 dims][32 keys] comes
// from LDS. The 32x32 accumulator holds 16 heads of one key per lane, so the
// ReLU head-sum is 16 in-lane adds plus one cross-half shuffle, and lanes
// 0..31 then hold 32 consecutive logits of a row.
#include "indexer_device.h"
#include "../../include/qsa_hip.h"

extern "C" __device__ unsigned int __ockl_wfred_max_u32(unsigned int);

namespace qsa {
namespace {

// ---------------------------------------------------------------------------
// Decode: grid (programs, rows), one wave per workgroup, TPW consecutive
// 16-key tiles per wave (kDecodeTilesWide, or kDecodeTilesNarrow when the wide
// split would leave compute units without a wave), logits to global memory.
// A row's waves stride over its visible keys, so the grid follows the batch,
// not the logits buffer's width: kDecodeTargetWaves waves over the batch
// (never more per row than the widest row needs), and a row longer than its
// waves cover in one pass takes several. The grid is (rows, programs), so
// every row's first programs are dispatched before any row's later ones:
// in a wide buffer the programs past a row's keys come last and exit while
// the others stream (64 rows of <= 2048 keys in the 32768-column class: 6.9
// us, against 11.3 us with programs innermost; 7.3 us in a 2048-column buffer).
//
// With D = 128 and a cache page of a multiple of 16 keys (DMA), the keys go
// straight into the wave's LDS as whole rows (score_tiles_dma): a CU's
// texture path streams four 256 B rows per instruction about twice as fast as
// the B operand's 16 keys x 64 B, which bounded the CUs holding several of a
// long row's waves (the programs of one row land on a few CUs of its XCD).
// decode_32k's indexer alone 6.87 -> 5.70 us; inside the decode step, where
// the keys come from HBM rather than the Infinity Cache, the step gains
// 0.2-0.3 us.
// ---------------------------------------------------------------------------
constexpr int kDecodeTilesWide = 8;
constexpr int kDecodeTilesNarrow = 4;
constexpr int kDecodeTargetWaves = 2048;

template <int D, int HB, int TPW, bool DMA = false>
__global__ __launch_bounds__(64) void indexer_decode_kernel(const IndexerParams p) {
  __shared__ __attribute__((aligned(16))) char s_keys[DMA ? TPW * kKeysPerTile * 256 : 16];
  const int row = blockIdx.x;
  const int program = blockIdx.y;
  const int programs = gridDim.y;
  const int num_columns = p.table_width * p.cache_page;
  const int vis = min(min(p.visible[row], num_columns), p.logits_cols);
  int tile0 = program * TPW;
  if (tile0 * kKeysPerTile >= vis) return;
  const int req = row / p.decode_query_len;
  const int32_t* trow = p.table + (int64_t)req * p.table_row;
  bf16x8 qa[HB][D / 32];
  load_q<D, HB>(p, row, qa);
  float* lrow = p.logits + (int64_t)row * p.logits_row;
  const int stride = programs * TPW;
  do {
    if constexpr (DMA)
      score_tiles_dma<HB, TPW>(p, trow, tile0, vis, qa, s_keys, [&](int c, float v) { lrow[c] = v; });
    else
      score_tiles<D, HB, TPW>(p, trow, tile0, vis, qa, [&](int c, float v) { lrow[c] = v; });
    tile0 += stride;
  } while (tile0 * kKeysPerTile < vis);
}

// ---------------------------------------------------------------------------
// Prefill: grid (32-row tiles of the call's rows, key chunks), 8 waves x 4
// rows. A tile's rows need not share a request: the workgroup makes one pass
// over the keys per request in the tile (a tile crossing a request boundary
// makes two). The grid depends only on the call's row count, so every
// launched workgroup has rows.
//
// Per 64-key tile, the workgroup stages the keys once in LDS (double
// buffered) and every wave multiplies them against its 4 rows' Q (held in
// registers for the whole chunk): 2 key blocks x 4 rows x 8 K steps = 64
// MFMAs per 8 KB B-operand read from LDS. The next tile's keys are loaded
// into registers while the current tile computes, and its page-table entries
// one tile earlier still, so the MFMAs never wait on a dependent load chain.
// One LDS-only barrier per tile keeps those loads in flight. All loads and
// stores are unconditional (invalid keys read the zero block, masked logits go
// to a discard slot) so every wait count is static.
// ---------------------------------------------------------------------------
constexpr int kPfRowsPerWave = 4;
constexpr int kPfWaves = 8;
constexpr int kPfThreads = 64 * kPfWaves;
constexpr int kPfRows = kPfRowsPerWave * kPfWaves;
constexpr int kPfTileKeys = 64;
constexpr int kPfHeads = 32;  // index-head slots of the A operand (M of the MFMA)
constexpr int kCUs = 256;     // compute units of an MI355X

// Sink for logits a lane must not write (columns past its row's visible
// count), shared by all lanes: keeps the store unconditional without a
// per-lane address register.
static __device__ float g_qsa_discard[1];

template <int D>
__global__ __launch_bounds__(kPfThreads) void indexer_prefill_kernel(const IndexerParams p) {
  constexpr int KS = D / 16;
  constexpr int ROW_BYTES = D * 2 + 16;                // padded: conflict-free 16 B reads
  constexpr int CH = D * 2 / 16;                       // 16 B chunks per key row
  constexpr int PER_THREAD = kPfTileKeys * CH / kPfThreads;
  static_assert(PER_THREAD * kPfThreads == kPfTileKeys * CH, "tile must split evenly");
  __shared__ __attribute__((aligned(16))) char s_keys[2][kPfTileKeys * ROW_BYTES];
  // One padded 32-head Q row per wave, for the Q layout change (below).
  __shared__ __attribute__((aligned(16))) char s_q[kPfWaves][kPfHeads * ROW_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int kk = lane & 31;
  const int half = lane >> 5;
  const int num_columns = p.table_width * p.cache_page;
  const int32_t* zero_i = reinterpret_cast<const int32_t*>(g_qsa_zero_rows);
  const char* zero = reinterpret_cast<const char*>(g_qsa_zero_rows);

  // The workgroup's 32 consecutive rows of this call's span. Later rows of a
  // request see more keys, so tiles go out last-first: the heaviest start
  // first and the short ones fill the end of the launch.
  const int row0 = p.query_offset + (int)(gridDim.x - 1 - blockIdx.x) * kPfRows;
  const int row_end = min(row0 + kPfRows, p.query_offset + p.num_rows);
  const int t_begin = blockIdx.y * p.key_tiles_per_wg;
  const int base = load_uniform(p.query_start_loc);

  // Request of row0: the last r with query_start_loc[r] - base <= row0 (the
  // last of any empty requests starting there is the one holding the row).
  int req = -1;
  for (int r0 = 0; r0 < p.num_requests; r0 += 64) {
    const int r = r0 + lane;
    const bool le = r < p.num_requests && p.query_start_loc[r] - base <= row0;
    const int n = __builtin_popcountll(__ballot(le));
    req += n;
    if (n < 64) break;
  }
  // The 32 rows take one pass over the keys per request they belong to (one,
  // unless the tile crosses a request boundary); in a pass, rows of other
  // requests see no keys.
  int seg_begin = row0;
  int seg_end = min(load_uniform(p.query_start_loc + req + 1) - base, row_end);
  if (seg_end <= seg_begin) return;

  // Pass state: the request's page-table row, the page entries of the next
  // two tiles to stage, the visible keys of the pass's rows and its tiles.
  const int32_t* trow;
  int pg_cur[PER_THREAD], pg_next[PER_THREAD];
  int rvis[kPfRowsPerWave];
  int wg_vis, t_end;
  // Page-table entries of this thread's staging keys (tid + kPfThreads j) /
  // CH of a tile, for every key inside the table: visibility is applied when
  // the keys are loaded, so the entries depend on the request alone.
  auto page_of = [&](int tile, int j) {
    const int c = tile * kPfTileKeys + (tid + kPfThreads * j) / CH;
    return *(c < num_columns ? trow + p.page_div.div(c) : zero_i);
  };
  // Issues the pass's page entries, then its visible counts (lane l of every
  // wave reads row l % 32, so each wave finds the workgroup maximum itself).
  auto setup_pass = [&]() {
    trow = p.table + (int64_t)req * p.table_row;
#pragma unroll
    for (int j = 0; j < PER_THREAD; ++j) pg_cur[j] = page_of(t_begin, j);
#pragma unroll
    for (int j = 0; j < PER_THREAD; ++j) pg_next[j] = page_of(t_begin + 1, j);
    const int vr = row0 + kk;
    const int my_vis = vr >= seg_begin && vr < seg_end
                           ? min(min(p.visible[vr], num_columns), p.logits_cols)
                           : 0;
    wg_vis = (int)__ockl_wfred_max_u32((uint32_t)my_vis);
#pragma unroll
    for (int i = 0; i < kPfRowsPerWave; ++i)
      rvis[i] = __builtin_amdgcn_readlane(my_vis, wave * kPfRowsPerWave + i);
    t_end = min(t_begin + p.key_tiles_per_wg, (wg_vis + kPfTileKeys - 1) / kPfTileKeys);
  };
  auto load_keys = [&](int tile, const int (&pg)[PER_THREAD], u32x4 (&st)[PER_THREAD]) {
#pragma unroll
    for (int j = 0; j < PER_THREAD; ++j) {
      const int e = tid + kPfThreads * j;
      const int c = tile * kPfTileKeys + e / CH;
      const int lp = p.page_div.div(c);
      const bool ok = c < wg_vis && pg[j] >= 0 && pg[j] < p.num_blocks;
      const char* kp = ok ? p.k + (int64_t)pg[j] * p.kb + (int64_t)(c - lp * p.cache_page) * p.kt
                          : zero;
      st[j] = load_u32x4(kp + (e % CH) * 16);
    }
  };
  auto store_keys = [&](int buf, const u32x4 (&st)[PER_THREAD]) {
#pragma unroll
    for (int j = 0; j < PER_THREAD; ++j) {
      const int e = tid + kPfThreads * j;
      *reinterpret_cast<u32x4*>(&s_keys[buf][(e / CH) * ROW_BYTES + (e % CH) * 16]) = st[j];
    }
  };

  // First pass prologue, in issue order: page entries, visible counts, Q,
  // the first tile's keys. A wave's vector loads complete in issue order, so
  // the visible counts wait for one round trip, and Q arrives with the keys.
  setup_pass();

  // Q of the wave's 4 rows. The A operand wants lane (kk, half) to hold head
  // kk, dims 16 s + 8 half .. +7: loaded directly, every load instruction
  // would touch 32 head rows for 32 bytes each, which measured ~13 us per
  // workgroup. Instead each 16-lane group (8 for D = 64) loads one head's
  // contiguous row, the wave writes the row into its padded LDS slot, and
  // reads it back in the A layout (the same conflict-free pattern as the
  // keys). Heads past num_heads and rows past the span are zeros.
  constexpr int HPL = 64 / CH;         // heads per load instruction
  constexpr int QLOADS = kPfHeads / HPL;
  static_assert(QLOADS == KS, "one Q load per K step of the A operand");
  const int qh0 = lane / CH;  // head of this lane in load n: n * HPL + qh0
  const int qc = lane % CH;   // 16 B chunk of that head's row
  bf16x8 qa[kPfRowsPerWave][KS];
#pragma unroll
  for (int i = 0; i < kPfRowsPerWave; ++i) {
    const int r = row0 + wave * kPfRowsPerWave + i;
    const uint16_t* qrow = p.q + (int64_t)r * p.q_row + qc * 8;
#pragma unroll
    for (int n = 0; n < QLOADS; ++n) {
      const int h = n * HPL + qh0;
      const bool ok = r < row_end && h < p.num_heads;
      qa[i][n] = __builtin_bit_cast(
          bf16x8, load_u32x4(ok ? (const void*)(qrow + (int64_t)h * p.q_head) : (const void*)zero));
    }
  }
  u32x4 st[PER_THREAD];
  load_keys(t_begin, pg_cur, st);
  {
    char* slot = s_q[wave];
#pragma unroll
    for (int i = 0; i < kPfRowsPerWave; ++i) {
#pragma unroll
      for (int n = 0; n < QLOADS; ++n)
        *reinterpret_cast<u32x4*>(slot + (n * HPL + qh0) * ROW_BYTES + qc * 16) =
            __builtin_bit_cast(u32x4, qa[i][n]);
      // A wave's LDS accesses complete in order: the reads see the row.
#pragma unroll
      for (int s2 = 0; s2 < KS; ++s2)
        qa[i][s2] = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const u32x4*>(slot + kk * ROW_BYTES + (16 * s2 + 8 * half) * 2));
    }
  }

  float* discard = g_qsa_discard;
  for (;;) {
    if (t_begin < t_end) {  // uniform across the workgroup
      store_keys(0, st);
      // Makes stage 0 visible; a previous pass ended at a barrier after its
      // last reads.
      lds_barrier();
      for (int tile = t_begin; tile < t_end; ++tile) {
        const int buf = (tile - t_begin) & 1;
        // Next tile's keys and the page entries of the one after.
        load_keys(tile + 1, pg_next, st);
#pragma unroll
        for (int j = 0; j < PER_THREAD; ++j) pg_next[j] = page_of(tile + 2, j);
        __builtin_amdgcn_sched_barrier(0);

        // The tile's (key block, row) products in order; the ReLU head-sum of
        // product j - 1 is interleaved with the MFMAs of product j (one MFMA,
        // then a few VALU ops), so each wave keeps the matrix pipe busy
        // through its own epilogues. Without that the per-tile barrier keeps
        // the two waves of a SIMD in step, and both leave the pipe idle
        // during their epilogues.
        constexpr int kBlocks = kPfTileKeys / 32;
        constexpr int kProducts = kBlocks * kPfRowsPerWave;
        bf16x8 kbf[2][KS];  // B operands of the current and previous key block
        f32x16 acc[2];
        // Rows are paired: lanes keep the ReLU head-sum of their 16 heads per
        // product, and one v_permlane32_swap of the pair's two partials gives
        // (partial_a, partial_b) = (a lo, b lo) and (a hi, b hi), whose sum
        // holds row i's 32 logits in lanes 0..31 and row i + 1's in lanes
        // 32..63: one swap, add and store per two products, every lane
        // storing a logit.
        static_assert(kPfRowsPerWave % 2 == 0, "rows are paired");
        float part[2];
        auto emit = [&](int j, const f32x16& a) {
          part[j & 1] = relu_head_sum(a);
          if ((j & 1) == 0) return;
          const int kb_i = j / kPfRowsPerWave;
          const int i = (j % kPfRowsPerWave) - 1 + half;  // this lane's row of the pair
          const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, part[0]),
                                                           __builtin_bit_cast(uint32_t, part[1]),
                                                           false, false);
          const float sum = __builtin_bit_cast(float, (uint32_t)sw[0]) +
                            __builtin_bit_cast(float, (uint32_t)sw[1]);
          const int c = tile * kPfTileKeys + kb_i * 32 + kk;
          const int r = row0 + wave * kPfRowsPerWave + i;
          const int vis = half ? rvis[(j % kPfRowsPerWave)] : rvis[(j % kPfRowsPerWave) - 1];
          float* dst =
              c < vis ? p.logits + (int64_t)(r - p.query_offset) * p.logits_row + c : discard;
          *dst = sum * p.scale;
        };
#pragma unroll
        for (int j = 0; j < kProducts; ++j) {
          const int kb_i = j / kPfRowsPerWave;
          const int i = j % kPfRowsPerWave;
          if (i == 0) {
            const char* krow = &s_keys[buf][(kb_i * 32 + kk) * ROW_BYTES];
#pragma unroll
            for (int s2 = 0; s2 < KS; ++s2)
              kbf[kb_i & 1][s2] = __builtin_bit_cast(
                  bf16x8, *reinterpret_cast<const u32x4*>(krow + (16 * s2 + 8 * half) * 2));
          }
          f32x16 a = {};
#pragma unroll
          for (int s2 = 0; s2 < KS; ++s2)
            a = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa[i][s2], kbf[kb_i & 1][s2], a, 0, 0, 0);
          acc[j & 1] = a;
          if (j > 0) emit(j - 1, acc[(j - 1) & 1]);
          if (i == 0) __builtin_amdgcn_sched_group_barrier(0x100, KS, 0);  // LDS reads first
#pragma unroll
          for (int s2 = 0; s2 < KS; ++s2) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);  // then VALU of the epilogue
          }
          __builtin_amdgcn_sched_barrier(0);
        }
        emit(kProducts - 1, acc[(kProducts - 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
        store_keys(buf ^ 1, st);
        lds_barrier();
      }
    }
    // The next request with rows in the tile, if any.
    seg_begin = seg_end;
    if (seg_begin >= row_end) break;
    do {
      ++req;
      if (req >= p.num_requests) return;
      seg_end = min(load_uniform(p.query_start_loc + req + 1) - base, row_end);
    } while (seg_end <= seg_begin);
    setup_pass();
    if (t_begin < t_end) load_keys(t_begin, pg_cur, st);
  }
}

// Key chunks of a prefill launch: one 8-wave workgroup fills a CU, so a
// launch of T row tiles runs in ceil(T * c / CUs) rounds of workgroups that
// each cover 1/c of the key range plus a fixed start (Q and the first tiles,
// ~12% of a whole-range workgroup). The count with the fewest such units
// wins: a whole number of rounds keeps whole key ranges (Q loaded once), a
// launch short of a round splits the keys to fill the chip.
int prefill_key_chunks(int64_t row_tiles, int max_tiles) {
  int best_c = 1;
  double best = 1e300;
  for (int c = 1; c <= std::min(8, std::max(1, max_tiles)); ++c) {
    const int64_t rounds = (row_tiles * c + kCUs - 1) / kCUs;
    const double cost = (double)rounds * (1.0 / c + 0.12);
    if (cost < best - 1e-9) {
      best = cost;
      best_c = c;
    }
  }
  return best_c;
}

int check_indexer(const void* q, int num_heads, int head_dim, const void* k_cache,
                  int cache_page, const int32_t* page_table, const int32_t* visible,
                  const float* logits, int64_t q_head_stride, int64_t q_row_stride,
                  int64_t cb, int64_t ct, const char* name) {
  if (!q || !k_cache || !page_table || !visible || !logits)
    return fail(QSA_ERR_INVALID, std::string(name) + ": null tensor pointer");
  if (head_dim != 64 && head_dim != 128)
    return fail(QSA_ERR_UNSUPPORTED, std::string(name) + ": head_dim must be 64 or 128");
  if (num_heads <= 0 || num_heads > 64)
    return fail(QSA_ERR_UNSUPPORTED, std::string(name) + ": num_heads must be in 1..64");
  if (cache_page <= 0) return fail(QSA_ERR_INVALID, std::string(name) + ": bad cache page size");
  if (((uintptr_t)q | (uintptr_t)k_cache) & 15u || (q_head_stride | q_row_stride | cb | ct) & 7)
    return fail(QSA_ERR_INVALID, std::string(name) +
                                     ": q/k_cache must be 16-byte aligned with strides that are "
                                     "multiples of 8 elements");
  return QSA_OK;
}

template <int T>
void launch_decode(const IndexerParams& p, int head_dim, int hb, dim3 grid, hipStream_t s) {
  if (head_dim == 128 && p.cache_page % kKeysPerTile == 0) {
    if (hb == 1) hipLaunchKernelGGL((indexer_decode_kernel<128, 1, T, true>), grid, dim3(64), 0, s, p);
    else if (hb == 2) hipLaunchKernelGGL((indexer_decode_kernel<128, 2, T, true>), grid, dim3(64), 0, s, p);
    else if (hb == 3) hipLaunchKernelGGL((indexer_decode_kernel<128, 3, T, true>), grid, dim3(64), 0, s, p);
    else hipLaunchKernelGGL((indexer_decode_kernel<128, 4, T, true>), grid, dim3(64), 0, s, p);
    return;
  }
  if (head_dim == 128) {
    if (hb == 1) hipLaunchKernelGGL((indexer_decode_kernel<128, 1, T>), grid, dim3(64), 0, s, p);
    else if (hb == 2) hipLaunchKernelGGL((indexer_decode_kernel<128, 2, T>), grid, dim3(64), 0, s, p);
    else if (hb == 3) hipLaunchKernelGGL((indexer_decode_kernel<128, 3, T>), grid, dim3(64), 0, s, p);
    else hipLaunchKernelGGL((indexer_decode_kernel<128, 4, T>), grid, dim3(64), 0, s, p);
  } else {
    if (hb == 1) hipLaunchKernelGGL((indexer_decode_kernel<64, 1, T>), grid, dim3(64), 0, s, p);
    else if (hb == 2) hipLaunchKernelGGL((indexer_decode_kernel<64, 2, T>), grid, dim3(64), 0, s, p);
    else if (hb == 3) hipLaunchKernelGGL((indexer_decode_kernel<64, 3, T>), grid, dim3(64), 0, s, p);
    else hipLaunchKernelGGL((indexer_decode_kernel<64, 4, T>), grid, dim3(64), 0, s, p);
  }
}

}  // namespace
}  // namespace qsa

using namespace qsa;

extern "C" int qsa_indexer_decode(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                                  int rows, int num_heads, int head_dim, const void* k_cache,
                                  int64_t cache_block_stride, int64_t cache_token_stride,
                                  int num_blocks, int cache_page, const int32_t* page_table,
                                  int64_t table_row_stride, int table_width,
                                  const int32_t* visible, int decode_query_len, float* logits,
                                  int64_t logits_row_stride, int logits_cols, void* stream) {
  if (rows < 0) return fail(QSA_ERR_INVALID, "qsa_indexer_decode: rows < 0");
  if (rows == 0 || logits_cols <= 0 || table_width <= 0) return QSA_OK;
  int st = check_indexer(q, num_heads, head_dim, k_cache, cache_page, page_table, visible, logits,
                         q_head_stride, q_row_stride, cache_block_stride, cache_token_stride,
                         "qsa_indexer_decode");
  if (st != QSA_OK) return st;
  if (decode_query_len <= 0) return fail(QSA_ERR_INVALID, "qsa_indexer_decode: decode_query_len");
  IndexerParams p = {};
  p.q = static_cast<const uint16_t*>(q);
  p.q_row = q_row_stride;
  p.q_head = q_head_stride;
  p.k = static_cast<const char*>(k_cache);
  p.kb = cache_block_stride * 2;
  p.kt = cache_token_stride * 2;
  p.num_blocks = num_blocks;
  p.cache_page = cache_page;
  p.page_div = FastDiv::make(cache_page);
  p.table = page_table;
  p.table_row = table_row_stride;
  p.table_width = table_width;
  p.visible = visible;
  p.num_heads = num_heads;
  p.decode_query_len = decode_query_len;
  p.logits = logits;
  p.logits_row = logits_row_stride;
  p.logits_cols = logits_cols;
  p.scale = (float)(1.0 / __builtin_sqrt((double)head_dim));
  // One wave per TPW key tiles of a row: every key of the batch is in flight
  // at once for batches up to tens of thousands of keys. Eight tiles per wave
  // halve the per-wave query loads and setup against four (MI355X, 32 x 128
  // index heads: 64 rows x 2048 keys 7.7 -> 7.2 us, 8 rows x up to 8192 keys
  // 4.71 -> 4.54 us; sixteen tiles need 256 registers and ran 8.1 / 6.1 us);
  // launches that would then leave compute units without a wave keep four.
  // Programs per row: kDecodeTargetWaves over the batch at most, never more
  // than the widest row of the buffer needs (the rows' own lengths are not
  // known on the host; a wide buffer's extra waves exit after one load).
  const int max_tiles = (std::min(logits_cols, table_width * cache_page) + kKeysPerTile - 1) /
                        kKeysPerTile;
  const int per_row = std::max(1, (kDecodeTargetWaves + rows - 1) / rows);
  const int wide_programs =
      std::max(1, std::min((max_tiles + kDecodeTilesWide - 1) / kDecodeTilesWide, per_row));
  const bool wide = (int64_t)wide_programs * rows >= kCUs;
  const int tpw = wide ? kDecodeTilesWide : kDecodeTilesNarrow;
  const int programs = std::max(1, std::min((max_tiles + tpw - 1) / tpw, per_row));
  const dim3 grid(rows, programs);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (programs > 65535) return fail(QSA_ERR_UNSUPPORTED, "qsa_indexer_decode: grid too large");
  // Head blocks of 16: up to 64 index heads.
  const int hb = (num_heads + 15) / 16;
  if (wide) launch_decode<kDecodeTilesWide>(p, head_dim, hb, grid, s);
  else launch_decode<kDecodeTilesNarrow>(p, head_dim, hb, grid, s);
  return check_launch("qsa_indexer_decode launch");
}

extern "C" int qsa_indexer_prefill(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                                   int num_heads, int head_dim, const void* k_cache,
                                   int64_t cache_block_stride, int64_t cache_token_stride,
                                   int num_blocks, int cache_page, const int32_t* page_table,
                                   int64_t table_row_stride, int table_width, int num_requests,
                                   const int32_t* query_start_loc, const int32_t* visible,
                                   int query_offset, int num_rows, int max_query_len,
                                   float* logits, int64_t logits_row_stride, int logits_cols,
                                   void* stream) {
  if (num_rows < 0 || num_requests < 0) return fail(QSA_ERR_INVALID, "qsa_indexer_prefill: negative shape");
  if (num_rows == 0 || num_requests == 0 || logits_cols <= 0 || table_width <= 0) return QSA_OK;
  int st = check_indexer(q, num_heads, head_dim, k_cache, cache_page, page_table, visible, logits,
                         q_head_stride, q_row_stride, cache_block_stride, cache_token_stride,
                         "qsa_indexer_prefill");
  if (st != QSA_OK) return st;
  if (num_heads > 32)
    return fail(QSA_ERR_UNSUPPORTED, "qsa_indexer_prefill: more than 32 index heads");
  if (!query_start_loc) return fail(QSA_ERR_INVALID, "qsa_indexer_prefill: null query_start_loc");
  IndexerParams p = {};
  p.q = static_cast<const uint16_t*>(q);
  p.q_row = q_row_stride;
  p.q_head = q_head_stride;
  p.k = static_cast<const char*>(k_cache);
  p.kb = cache_block_stride * 2;
  p.kt = cache_token_stride * 2;
  p.num_blocks = num_blocks;
  p.cache_page = cache_page;
  p.page_div = FastDiv::make(cache_page);
  p.table = page_table;
  p.table_row = table_row_stride;
  p.table_width = table_width;
  p.visible = visible;
  p.num_heads = num_heads;
  p.decode_query_len = 1;
  p.logits = logits;
  p.logits_row = logits_row_stride;
  p.logits_cols = logits_cols;
  p.scale = (float)(1.0 / __builtin_sqrt((double)head_dim));
  p.query_start_loc = query_start_loc;
  p.num_requests = num_requests;
  p.query_offset = query_offset;
  p.num_rows = num_rows;
  (void)max_query_len;  // the launch tiles this call's rows, whatever the requests' lengths
  const int64_t row_tiles = ((int64_t)num_rows + kPfRows - 1) / kPfRows;
  const int max_tiles = (std::min(logits_cols, table_width * cache_page) + kPfTileKeys - 1) /
                        kPfTileKeys;
  const int key_chunks = prefill_key_chunks(row_tiles, max_tiles);
  p.key_tiles_per_wg = std::max(1, (std::max(1, max_tiles) + key_chunks - 1) / key_chunks);
  if (row_tiles > INT32_MAX)
    return fail(QSA_ERR_UNSUPPORTED, "qsa_indexer_prefill: grid too large");
  const dim3 grid((unsigned)row_tiles, (unsigned)key_chunks);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (head_dim == 128)
    hipLaunchKernelGGL((indexer_prefill_kernel<128>), grid, dim3(kPfThreads), 0, s, p);
  else
    hipLaunchKernelGGL((indexer_prefill_kernel<64>), grid, dim3(kPfThreads), 0, s, p);
  return check_launch("qsa_indexer_prefill launch");
}

extern "C" int qsa_indexer_prefill_span_rows(int logits_cols, int64_t cap_bytes) {
  if (logits_cols <= 0) return 1;
  const int64_t cap_rows = std::max<int64_t>(1, cap_bytes / (4 * (int64_t)logits_cols));
  // Whole rounds of one 32-row workgroup per CU when the cap allows one.
  const int64_t round_rows = (int64_t)kCUs * kPfRows;
  const int64_t rows = cap_rows >= round_rows ? cap_rows / round_rows * round_rows : cap_rows;
  return (int)std::min<int64_t>(rows, INT32_MAX);
}
