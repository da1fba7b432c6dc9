// Kernel 2: exact per-row top-k block selection + token expansion, gfx950.
//
// Semantics and algorithm: topk_device.h. This file holds the kernels (direct,
// and partition + merge for rows longer than the register-resident capacity)
// and the C ABI entry points.
#include "topk_device.h"
#include "../../include/qsa_hip.h"

namespace qsa {
namespace {

// --- kernels ---------------------------------------------------------------

// Rows at which the chip is full and throughput, not one row's latency, sets
// the time (the launch shapes switch there), and rows beyond which the
// narrowest shapes win for rows of up to 2048 columns.
constexpr int kManyRows = 1024;
constexpr int kFullChipRows = 4096;

struct TopkArgs {
  const float* scores;
  int64_t score_row_stride;
  const int32_t* lengths;
  int32_t* out;
  int64_t out_row_stride;
  int32_t* partial;  // [rows, parts, topk] for the two-pass path
  int parts;
  int topk;
  int cols;  // row width: lengths beyond it are clamped so no read leaves the row
  ExpandMeta meta;
};

// Rows longer than k are scored from the logits row, so their length is
// clamped to the row width (a longer length reads past the row in the
// reference). Rows of at most k entries only emit ids and keep their length.
__device__ __forceinline__ int row_length(const TopkArgs& a, int row) {
  const int length = a.lengths[row];
  return length > a.topk ? min(length, a.cols) : length;
}

// The selected ids (2 * topk ints) share LDS with the key stage when they fit
// in it (the stage is dead by then); otherwise they get dynamic LDS.
template <int THREADS, int ITEMS>
constexpr bool sel_in_stage(int topk) { return 2 * topk <= THREADS * ITEMS; }

#define QSA_TOPK_LDS(THREADS, ITEMS, PAGES)              \
  __shared__ TopkShared<THREADS> sh;                     \
  __shared__ TopkStage<THREADS, ITEMS, PAGES> st;        \
  extern __shared__ int dyn_sel[];                       \
  int* sel = sel_in_stage<THREADS, ITEMS>(a.topk) ? reinterpret_cast<int*>(st.key) : dyn_sel

template <int THREADS, int ITEMS, bool EXPAND, bool PAGES>
__global__ __launch_bounds__(THREADS) void topk_direct_kernel(const TopkArgs a) {
  QSA_TOPK_LDS(THREADS, ITEMS, PAGES);
  const int row = blockIdx.x;
  const float* srow = a.scores + (int64_t)row * a.score_row_stride;
  process_row_whole<THREADS, ITEMS, EXPAND, PAGES>(DirectLoader{srow, 0}, a.cols, a.lengths[row],
                                                   a.cols, a.topk, a.meta, row,
                                                   a.out + (int64_t)row * a.out_row_stride, sh,
                                                   st, sel);
}

// Pass 1 of long rows: rows short enough for one pass finish in partition 0.
template <int THREADS, int ITEMS, bool EXPAND, bool PAGES>
__global__ __launch_bounds__(THREADS) void topk_partition_kernel(const TopkArgs a) {
  QSA_TOPK_LDS(THREADS, ITEMS, PAGES);
  const int row = blockIdx.x;
  const int part = blockIdx.y;
  const int length = row_length(a, row);
  const float* srow = a.scores + (int64_t)row * a.score_row_stride;
  if (length <= kPartitionColumns) {
    if (part == 0)
      process_row<THREADS, ITEMS, EXPAND, PAGES>(DirectLoader{srow, 0}, length, length, length,
                                                 a.topk, a.meta, row,
                                                 a.out + (int64_t)row * a.out_row_stride, sh, st, sel);
    return;
  }
  const int start = part * kPartitionColumns;
  if (start >= length) return;
  const int count = min(kPartitionColumns, length - start);
  int32_t* prow = a.partial + ((int64_t)row * a.parts + part) * a.topk;
  process_row<THREADS, ITEMS, false, false>(DirectLoader{srow, start}, count, count, count, a.topk,
                                            a.meta, row, prow, sh, st, sel);
}

// Pass 2: exact top-k over the concatenated partition winners (ascending ids).
template <int THREADS, int ITEMS, bool EXPAND, bool PAGES>
__global__ __launch_bounds__(THREADS) void topk_merge_kernel(const TopkArgs a) {
  QSA_TOPK_LDS(THREADS, ITEMS, PAGES);
  const int row = blockIdx.x;
  const int length = row_length(a, row);
  if (length <= kPartitionColumns) return;
  const int count = (length / kPartitionColumns) * a.topk + min(length % kPartitionColumns, a.topk);
  const float* srow = a.scores + (int64_t)row * a.score_row_stride;
  const IndirectLoader load{srow, a.partial + (int64_t)row * a.parts * a.topk};
  process_row<THREADS, ITEMS, EXPAND, PAGES>(load, count, count, count, a.topk, a.meta, row,
                                             a.out + (int64_t)row * a.out_row_stride, sh, st, sel);
}

// Few rows of a wide logits buffer (a decode batch in a wide width class):
// one 1024-thread workgroup per row sizes its keys per thread by the row's
// own length (2, 4, 8 or 16, and enough that the selection fits the dead key
// stage), so a row costs what its length needs, whatever the buffer's width.
// A row of 16385..32768 keys takes exact top-k of its two halves in turn
// (winners kept in LDS), then exact top-k over the halves' winners in id
// order. One static LDS region serves every shape: 16 keys per thread and
// their pages, or the halves' keys and winners.
constexpr int kAdaptiveThreads = 1024;
constexpr int kAdaptiveHalf = kAdaptiveThreads * 16;
constexpr int kAdaptiveMaxColumns = 2 * kAdaptiveHalf;

// Rows of up to this many threads x 4 keys (2048) run on the lower waves
// alone, in the 512 x 4 shape of the direct kernel for 2048 columns.
constexpr int kAdaptiveNarrow = 512;

template <bool EXPAND, bool PAGES>
__global__ __launch_bounds__(kAdaptiveThreads) void topk_adaptive_kernel(const TopkArgs a) {
  constexpr int T = kAdaptiveThreads;
  __shared__ union {
    TopkShared<T> full;
    TopkShared<kAdaptiveNarrow> narrow;
  } shu;
  auto& sh = shu.full;
  __shared__ __attribute__((aligned(16))) uint32_t stage_mem[T * 16 * 2];
  const int row = blockIdx.x;
  const float* srow = a.scores + (int64_t)row * a.score_row_stride;
  int32_t* out = a.out + (int64_t)row * a.out_row_stride;
  const int topk = a.topk;
  // Rows of up to kNarrowCols keys (the usual decode batch in a wide class)
  // run on the lower waves in the 512 x 4 shape. Their loads go out before
  // the row's length is known (the first min(kNarrowCols, cols) columns, all
  // inside the row; the launch gives this kernel rows of more than
  // kNarrowCols columns), so a short row waits for one round trip instead of
  // the length's and then its scores'.
  constexpr int kNarrowCols = kAdaptiveNarrow * 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform branches
  if (wave < kAdaptiveNarrow / 64 && 2 * topk <= kNarrowCols) {
    const DirectLoader load{srow, 0};
    const int limit = min(kNarrowCols, a.cols);
    uint32_t v[4];
    int pg[4];
    const RowPrefetch f =
        load_row<kAdaptiveNarrow, 4, EXPAND, PAGES>(load, limit, a.meta, row, v, pg);
    // Nothing below may wait for the length before the loads above are out.
    __builtin_amdgcn_sched_barrier(0);
    const int length = a.lengths[row];
    if (min(length, a.cols) <= kNarrowCols) {  // n <= kNarrowCols
      auto& st = *reinterpret_cast<TopkStage<kAdaptiveNarrow, 4, PAGES>*>(stage_mem);
      process_loaded_whole<kAdaptiveNarrow, 4, EXPAND, PAGES, false>(
          load, limit, v, pg, [&] { return f; }, length, a.cols, topk, a.meta, row, out,
          shu.narrow, st, reinterpret_cast<int*>(st.key));
      return;
    }
  }
  const int length = a.lengths[row];
  const int n = min(max(length, 0), a.cols);
#define QSA_ADAPTIVE_ROW(ITEMS, LOAD, LIMIT, LENGTH, CLAMP)                                     \
  {                                                                                             \
    auto& st = *reinterpret_cast<TopkStage<T, ITEMS, PAGES>*>(stage_mem);                      \
    static_assert(sizeof(TopkStage<T, ITEMS, PAGES>) <= sizeof(stage_mem), "stage too large");  \
    process_row<T, ITEMS, EXPAND, PAGES>(LOAD, LIMIT, LENGTH, CLAMP, topk, a.meta, row, out, sh, \
                                         st, reinterpret_cast<int*>(st.key));                   \
  }
#define QSA_ADAPTIVE_WHOLE_ROW(ITEMS)                                                           \
  {                                                                                             \
    auto& st = *reinterpret_cast<TopkStage<T, ITEMS, PAGES>*>(stage_mem);                      \
    static_assert(sizeof(TopkStage<T, ITEMS, PAGES>) <= sizeof(stage_mem), "stage too large");  \
    process_row_whole<T, ITEMS, EXPAND, PAGES>(load, n, length, a.cols, topk, a.meta, row, out, \
                                               sh, st, reinterpret_cast<int*>(st.key));         \
  }
  if (n <= kAdaptiveHalf) {
    const DirectLoader load{srow, 0};
    // Keys, and room for the selection. Rows of up to 4096 keys take four
    // per thread, so the candidates the bound leaves are compacted to one per
    // thread.
    const int need = max(n, 2 * topk);
    // A short row was selected above by the lower waves; the upper waves end
    // here. A barrier waits only for the waves of the workgroup that have not
    // ended, so the lower half runs the 512-thread row with its own barriers;
    // fewer waves per barrier and per block scan make each phase of a short
    // row cheaper.
    if (need <= kNarrowCols) return;
    if (need <= T * 4) QSA_ADAPTIVE_WHOLE_ROW(4)
    else if (need <= T * 8) QSA_ADAPTIVE_WHOLE_ROW(8)
    else QSA_ADAPTIVE_WHOLE_ROW(16)
    return;
  }
  // Halves: [0, 16384) and [16384, n), winners (ascending ids) to LDS past the
  // halves' key stage; the second half's candidates follow the first's, so
  // the merged list is in id order (ties go to the lower id, as in one pass).
  int* winners = reinterpret_cast<int*>(stage_mem + T * 16);
  auto& hst = *reinterpret_cast<TopkStage<T, 16, false>*>(stage_mem);
  int* hsel = reinterpret_cast<int*>(hst.key);
  process_row<T, 16, false, false>(DirectLoader{srow, 0}, kAdaptiveHalf, kAdaptiveHalf,
                                   kAdaptiveHalf, topk, a.meta, row, winners, sh, hst, hsel);
  __syncthreads();
  const int rest = n - kAdaptiveHalf;
  process_row<T, 16, false, false>(DirectLoader{srow, kAdaptiveHalf}, rest, rest, rest, topk,
                                   a.meta, row, winners + topk, sh, hst, hsel);
  __syncthreads();
  const int count = topk + min(rest, topk);
  const IndirectLoader merged{srow, winners};
  // Each thread reads its candidates' ids before it overwrites the same LDS
  // words with their pages (the page half of a 16-key stage is the winners).
  const int need = max(count, 2 * topk);
  if (need <= T * 2) QSA_ADAPTIVE_ROW(2, merged, count, count, count)
  else if (need <= T * 4) QSA_ADAPTIVE_ROW(4, merged, count, count, count)
  else if (need <= T * 8) QSA_ADAPTIVE_ROW(8, merged, count, count, count)
  else QSA_ADAPTIVE_ROW(16, merged, count, count, count)
#undef QSA_ADAPTIVE_ROW
#undef QSA_ADAPTIVE_WHOLE_ROW
}

template <int THREADS, int ITEMS>
size_t dyn_lds(int topk) {
  return sel_in_stage<THREADS, ITEMS>(topk) ? 0 : (size_t)2 * topk * sizeof(int);
}

template <int THREADS, int ITEMS, bool EXPAND>
hipError_t launch_direct(const TopkArgs& a, int rows, hipStream_t s) {
  const size_t lds = dyn_lds<THREADS, ITEMS>(a.topk);
  if (EXPAND && a.meta.physical)
    hipLaunchKernelGGL((topk_direct_kernel<THREADS, ITEMS, true, true>), dim3(rows), dim3(THREADS),
                       lds, s, a);
  else
    hipLaunchKernelGGL((topk_direct_kernel<THREADS, ITEMS, EXPAND, false>), dim3(rows),
                       dim3(THREADS), lds, s, a);
  return hipGetLastError();
}

int partitions_for(int cols) { return (cols + kPartitionColumns - 1) / kPartitionColumns; }

template <bool EXPAND>
int launch_topk(TopkArgs a, int rows, int cols, void* workspace, size_t workspace_bytes,
                hipStream_t s) {
  if (rows == 0) return QSA_OK;
  if (a.topk > kMaxTopk)
    return fail(QSA_ERR_UNSUPPORTED, "qsa_topk: more than 8192 selected blocks per row");
  hipError_t err;
  if (rows < kManyRows && cols > 2048 && cols <= kAdaptiveMaxColumns) {
    // A decode batch (latency-bound: one workgroup per row) over a buffer
    // wider than the 2048 columns the fixed shapes below are tuned for: the
    // buffer's width is its width class, not its rows' lengths (a 32768-column
    // class holds rows of 512-2048 keys at 8k-32k contexts), so each row sizes
    // its own work.
    const bool pages = EXPAND && a.meta.physical;
    if (pages)
      hipLaunchKernelGGL((topk_adaptive_kernel<true, true>), dim3(rows), dim3(kAdaptiveThreads), 0,
                         s, a);
    else
      hipLaunchKernelGGL((topk_adaptive_kernel<EXPAND, false>), dim3(rows),
                         dim3(kAdaptiveThreads), 0, s, a);
    if ((err = hipGetLastError()) != hipSuccess)
      return fail(QSA_ERR_HIP, std::string("qsa_topk launch: ") + hipGetErrorString(err));
    return QSA_OK;
  }
  if (cols <= kMaxDirectColumns) {
    // Few rows (a decode batch) leave most CUs idle and the time is one row's
    // latency: wider workgroups shorten the per-thread serial parts
    // (histogram updates, rank emission). Measured on 64 rows, top 128 with
    // physical expansion: 1024 columns 512 x 2 6.6 us (1024 x 2 7.5, 256 x 4
    // 8.0); 2048 columns 512 x 4 7.9 us (1024 x 2 8.1, 1024 x 4 8.6); 4096
    // columns 1024 x 4 10.0 us (512 x 8 9.9); 8192 columns 1024 x 8 13.1 us
    // (512 x 16 14.8). Many rows fill the chip and the time is throughput:
    // narrower workgroups do less redundant per-workgroup work (rows of random
    // length up to the width: 32768 x 1536 256 x 8 0.26 ms, 512 x 4 0.31 ms;
    // 32768 x 1024 256 x 4 0.18 ms, 512 x 2 0.27 ms), while up to about two
    // thousand rows 512 x 4 still wins (1024 x 2048: 16.8 us, 256 x 8 18.0).
    const bool latency_bound = rows < kManyRows;
    if (cols <= 1024 && latency_bound) err = launch_direct<512, 2, EXPAND>(a, rows, s);
    else if (cols <= 1024) err = launch_direct<256, 4, EXPAND>(a, rows, s);
    else if (cols <= 2048 && rows < kFullChipRows) err = launch_direct<512, 4, EXPAND>(a, rows, s);
    else if (cols <= 2048) err = launch_direct<256, 8, EXPAND>(a, rows, s);
    else if (cols <= 4096 && latency_bound) err = launch_direct<1024, 4, EXPAND>(a, rows, s);
    else if (cols <= 4096) err = launch_direct<512, 8, EXPAND>(a, rows, s);
    else if (cols <= 8192) err = launch_direct<1024, 8, EXPAND>(a, rows, s);
    else err = launch_direct<1024, 16, EXPAND>(a, rows, s);
    if (err != hipSuccess) return fail(QSA_ERR_HIP, std::string("qsa_topk launch: ") + hipGetErrorString(err));
    return QSA_OK;
  }
  const int parts = partitions_for(cols);
  if ((int64_t)parts * a.topk > kMaxDirectColumns)
    return fail(QSA_ERR_UNSUPPORTED, "qsa_topk: partition winners exceed 16384 candidates");
  if (a.topk > kPartitionColumns)
    return fail(QSA_ERR_UNSUPPORTED, "qsa_topk: topk above 8192 with rows above 16384 columns");
  const size_t need = (size_t)rows * parts * a.topk * sizeof(int32_t);
  if (!workspace || workspace_bytes < need)
    return fail(QSA_ERR_WORKSPACE, "qsa_topk: workspace too small for partition winners");
  a.partial = static_cast<int32_t*>(workspace);
  a.parts = parts;
  const bool pages = EXPAND && a.meta.physical;
  if (pages)
    hipLaunchKernelGGL((topk_partition_kernel<1024, 8, true, true>), dim3(rows, parts), dim3(1024),
                       (dyn_lds<1024, 8>(a.topk)), s, a);
  else
    hipLaunchKernelGGL((topk_partition_kernel<1024, 8, EXPAND, false>), dim3(rows, parts),
                       dim3(1024), (dyn_lds<1024, 8>(a.topk)), s, a);
  if ((err = hipGetLastError()) != hipSuccess)
    return fail(QSA_ERR_HIP, std::string("qsa_topk partition launch: ") + hipGetErrorString(err));
  if (pages)
    hipLaunchKernelGGL((topk_merge_kernel<1024, 16, true, true>), dim3(rows), dim3(1024),
                       (dyn_lds<1024, 16>(a.topk)), s, a);
  else
    hipLaunchKernelGGL((topk_merge_kernel<1024, 16, EXPAND, false>), dim3(rows), dim3(1024),
                       (dyn_lds<1024, 16>(a.topk)), s, a);
  if ((err = hipGetLastError()) != hipSuccess)
    return fail(QSA_ERR_HIP, std::string("qsa_topk merge launch: ") + hipGetErrorString(err));
  return QSA_OK;
}

// Expansion of caller-chosen block ids (expand_qsa_block_indices_cuda,
// ops/qsa.py:18-106, 552-591): rank i < topk is block_indices[row, i], in the
// caller's order; everything else as in topk_expand's writer.
struct ExpandBlocksArgs {
  const int32_t* blocks;
  int64_t block_row_stride, block_col_stride;
  int32_t* out;
  int64_t out_row_stride;
  int topk;
  ExpandMeta meta;
};

constexpr int kExpandThreads = 256;

__global__ __launch_bounds__(kExpandThreads) void expand_blocks_kernel(const ExpandBlocksArgs a) {
  __shared__ int tail_page[kTailSlots];
  extern __shared__ int sel[];  // block ids, then their first tokens' slots
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const RowPrefetch f =
      prefetch_tail<true>(a.meta, a.meta.token_to_req[row], (int)a.meta.positions[row]);
  const int32_t* brow = a.blocks + (int64_t)row * a.block_row_stride;
  for (int i = tid; i < a.topk; i += kExpandThreads) {
    const int b = brow[(int64_t)i * a.block_col_stride];
    sel[i] = b;
    sel[a.topk + i] =
        (a.meta.physical && b >= 0) ? first_slot(a.meta, block_page(a.meta, f.r, b, true), b) : -1;
  }
  if (tid < kTailSlots && tid < a.meta.ratio - 1) tail_page[tid] = f.tail_ok ? f.tail_pp : -1;
  lds_barrier();
  write_expanded(a.meta, f.r, row, a.topk, sel, tail_page, a.out + (int64_t)row * a.out_row_stride,
                 kExpandThreads);
}

int check_common(const float* scores, int rows, int cols, const int32_t* lengths,
                 const int32_t* output, int topk, const char* name) {
  if (rows < 0 || cols < 0) return fail(QSA_ERR_INVALID, std::string(name) + ": negative shape");
  if (rows == 0) return QSA_OK;
  if (!scores || !lengths || !output)
    return fail(QSA_ERR_INVALID, std::string(name) + ": null tensor pointer");
  if (topk <= 0) return fail(QSA_ERR_INVALID, std::string(name) + ": topk must be positive");
  return QSA_OK;
}

}  // namespace
}  // namespace qsa

using namespace qsa;

extern "C" size_t qsa_topk_workspace_bytes(int rows, int cols, int topk) {
  if (rows <= 0 || cols <= kMaxDirectColumns || topk <= 0) return 0;
  if (rows < kManyRows && cols <= kAdaptiveMaxColumns) return 0;  // one workgroup per row
  return (size_t)rows * partitions_for(cols) * topk * sizeof(int32_t);
}

extern "C" int qsa_topk(const float* scores, int64_t score_row_stride, int rows, int cols,
                        const int32_t* lengths, int32_t* output, int64_t output_row_stride,
                        int topk, void* workspace, size_t workspace_bytes, void* stream) {
  int st = check_common(scores, rows, cols, lengths, output, topk, "qsa_topk");
  if (st != QSA_OK || rows == 0) return st;
  TopkArgs a = {};
  a.scores = scores;
  a.score_row_stride = score_row_stride;
  a.lengths = lengths;
  a.out = output;
  a.out_row_stride = output_row_stride;
  a.topk = topk;
  a.cols = cols;
  a.meta.ratio = 1;
  a.meta.ratio_div = FastDiv::make(1);
  a.meta.page_size = 1;
  a.meta.page_div = FastDiv::make(1);
  return launch_topk<false>(a, rows, cols, workspace, workspace_bytes,
                            static_cast<hipStream_t>(stream));
}

namespace qsa {
namespace {

int topk_expand(const float* scores, int64_t score_row_stride, int rows, int cols,
                const int32_t* lengths, const int64_t* positions, const int32_t* sequence_lengths,
                int num_requests, const int32_t* token_to_req, const int32_t* table,
                int64_t table_row_stride, int table_width, int32_t* output,
                int64_t output_row_stride, int64_t output_col_stride, int output_width,
                int32_t* counts, int ratio, int page_size, int physical, int store_counts,
                void* workspace, size_t workspace_bytes, void* stream, const char* name) {
  if (ratio <= 0) return fail(QSA_ERR_INVALID, std::string(name) + ": ratio must be positive");
  const int topk = output_width / ratio;
  int st = check_common(scores, rows, cols, lengths, output, topk, name);
  if (st != QSA_OK || rows == 0) return st;
  if (!positions || !sequence_lengths || !token_to_req)
    return fail(QSA_ERR_INVALID, std::string(name) + ": null metadata pointer");
  if (physical && (!table || page_size <= 0))
    return fail(QSA_ERR_INVALID,
                std::string(name) + ": physical mapping needs a table and page_size");
  if (store_counts && !counts) return fail(QSA_ERR_INVALID, std::string(name) + ": null counts");
  TopkArgs a = {};
  a.scores = scores;
  a.score_row_stride = score_row_stride;
  a.lengths = lengths;
  a.out = output;
  a.out_row_stride = output_row_stride;
  a.topk = topk;
  a.cols = cols;
  a.meta = make_expand_meta(positions, sequence_lengths, num_requests, token_to_req, table,
                            table_row_stride, table_width, counts, output_col_stride,
                            output_width, ratio, page_size, physical, store_counts);
  return launch_topk<true>(a, rows, cols, workspace, workspace_bytes,
                           static_cast<hipStream_t>(stream));
}

}  // namespace
}  // namespace qsa

extern "C" int qsa_topk_expand(const float* scores, int64_t score_row_stride, int rows, int cols,
                               const int32_t* lengths, const int64_t* positions,
                               const int32_t* sequence_lengths, int num_requests,
                               const int32_t* token_to_req, const int32_t* table,
                               int64_t table_row_stride, int table_width, int32_t* output,
                               int64_t output_row_stride, int64_t output_col_stride,
                               int output_width, int32_t* counts, int ratio, int page_size,
                               int physical, int store_counts, void* workspace,
                               size_t workspace_bytes, void* stream) {
  return topk_expand(scores, score_row_stride, rows, cols, lengths, positions, sequence_lengths,
                     num_requests, token_to_req, table, table_row_stride, table_width, output,
                     output_row_stride, output_col_stride, output_width, counts, ratio, page_size,
                     physical, store_counts, workspace, workspace_bytes, stream,
                     "qsa_topk_expand");
}

extern "C" int qsa_expand_block_indices(const int32_t* block_indices, int64_t block_row_stride,
                                        int64_t block_col_stride, int block_cols, int rows,
                                        int topk, const int64_t* positions,
                                        const int32_t* sequence_lengths, int num_requests,
                                        const int32_t* token_to_req, const int32_t* table,
                                        int64_t table_row_stride, int table_width,
                                        int32_t* output, int64_t output_row_stride,
                                        int64_t output_col_stride, int output_width,
                                        int32_t* counts, int ratio, int page_size, int physical,
                                        int store_counts, void* stream) {
  if (rows < 0) return fail(QSA_ERR_INVALID, "qsa_expand_block_indices: negative rows");
  if (rows == 0) return QSA_OK;
  if (ratio <= 0 || topk <= 0 || topk > kMaxTopk)
    return fail(QSA_ERR_INVALID, "qsa_expand_block_indices: ratio and topk must be positive "
                                 "(topk at most 8192)");
  if (block_cols < topk)
    return fail(QSA_ERR_INVALID, "qsa_expand_block_indices: fewer block columns than topk");
  if (!block_indices || !positions || !sequence_lengths || !token_to_req || !output)
    return fail(QSA_ERR_INVALID, "qsa_expand_block_indices: null tensor pointer");
  if (physical && (!table || page_size <= 0))
    return fail(QSA_ERR_INVALID,
                "qsa_expand_block_indices: physical mapping needs a table and page_size");
  if (store_counts && !counts) return fail(QSA_ERR_INVALID, "qsa_expand_block_indices: null counts");
  ExpandBlocksArgs a = {};
  a.blocks = block_indices;
  a.block_row_stride = block_row_stride;
  a.block_col_stride = block_col_stride;
  a.out = output;
  a.out_row_stride = output_row_stride;
  a.topk = topk;
  a.meta.positions = positions;
  a.meta.sequence_lengths = sequence_lengths;
  a.meta.token_to_req = token_to_req;
  a.meta.table = physical ? table : nullptr;
  a.meta.counts = counts;
  a.meta.table_row_stride = table_row_stride;
  a.meta.out_col_stride = output_col_stride;
  a.meta.num_requests = num_requests;
  a.meta.table_width = physical ? table_width : 0;
  a.meta.page_size = page_size > 0 ? page_size : 1;
  a.meta.page_div = FastDiv::make(page_size > 0 ? page_size : 1);
  a.meta.ratio = ratio;
  a.meta.ratio_div = FastDiv::make(ratio);
  a.meta.out_width = output_width;
  a.meta.physical = physical ? 1 : 0;
  a.meta.store_counts = store_counts ? 1 : 0;
  hipLaunchKernelGGL(expand_blocks_kernel, dim3(rows), dim3(kExpandThreads),
                     (size_t)2 * topk * sizeof(int), static_cast<hipStream_t>(stream), a);
  return check_launch("qsa_expand_block_indices launch");
}
