// Kernel 2: exact per-row top-k block selection + token expansion, gfx950.
//
// Semantics follow ops/csrc/topk.cu of the reference plugin:
//  * order key = raw fp32 bit pattern read as uint32 (topk.cu:262, 331-338),
//    larger key first, lower id first among equal keys;
//  * rows with length <= k emit ids 0..length-1 then -1 (topk.cu:187-191);
//  * selected ids are emitted in ascending id order (topk.cu:328-349);
//  * expansion, causal tail, physical slot mapping and counts as
//    ExpandedWriter (topk.cu:97-180).
//
// Algorithm (own design for wave64 + LDS): one workgroup per row holds the
// row's keys in registers (blocked: thread t owns ids [t*ITEMS, t*ITEMS+ITEMS)).
// A radix select narrows the candidate set 8 bits at a time, always starting
// at the highest bit in which the remaining candidates still differ (found by a
// block min/max), so clustered scores do not waste passes on a shared prefix.
// Histograms use LDS atomics with a wave-uniform fast path. When the candidate
// range collapses to one key T, the selected set is {key > T} plus the first
// `remaining` ids with key == T, and a block-wide exclusive scan of
// (count > T, count == T) in id order gives every selected id its output rank.
// Rows longer than the register-resident capacity use two passes: exact top-k
// per 8192-column partition, then exact top-k over the partition winners.
#include "qsa_common.h"
#include "../../include/qsa_hip.h"

namespace qsa {
namespace {

constexpr int kPartitionColumns = 8192;
constexpr int kMaxDirectColumns = 16384;  // register-resident capacity: 1024 threads x 16 keys

template <int THREADS>
struct SelectShared {
  uint32_t hist[256];
  uint32_t wmin[THREADS / 64];
  uint32_t wmax[THREADS / 64];
  int wgt[THREADS / 64];
  int weq[THREADS / 64];
  int bin;
  int remaining;
};

// --- writers ---------------------------------------------------------------

struct CompressedWriter {  // topk.cu:90-95
  int32_t* out;
  __device__ __forceinline__ void operator()(int rank, int id) const { out[rank] = id; }
  __device__ __forceinline__ void finish() const {}
};

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
  int out_width;
  int physical;
  int store_counts;
};

struct ExpandWriter {  // topk.cu:107-180
  int32_t* out;
  int32_t* count;
  const int32_t* table_row;
  int64_t col_stride;
  int seq_len, complete, tail_start, tail_count;
  int page_size, table_width, ratio, out_width;
  FastDiv page_div;
  bool physical;

  __device__ __forceinline__ int map_token(int t) const {
    if (t < 0 || t >= seq_len) return -1;
    if (!physical) return t;
    const int lp = page_div.div(t);
    if (lp >= table_width) return -1;
    const int pp = table_row[lp];
    return pp >= 0 ? pp * page_size + (t - lp * page_size) : -1;
  }

  __device__ __forceinline__ void operator()(int rank, int block) const {
    if (rank >= complete) return;
    const int first = block * ratio;
    int32_t* dst = out + (int64_t)rank * ratio * col_stride;
    if (physical && page_size % ratio == 0) {
      // The block lies inside one page: one table lookup serves all members.
      int first_slot = -1;
      if (first >= 0 && first < seq_len) {
        const int lp = page_div.div(first);
        const int pp = lp < table_width ? table_row[lp] : -1;
        if (pp >= 0) first_slot = pp * page_size + (first - lp * page_size);
      }
      for (int o = 0; o < ratio; ++o)
        dst[(int64_t)o * col_stride] = (first_slot >= 0 && first + o < seq_len) ? first_slot + o : -1;
      return;
    }
    for (int o = 0; o < ratio; ++o) dst[(int64_t)o * col_stride] = map_token(first + o);
  }

  __device__ __forceinline__ void finish() const {
    const int expanded = complete * ratio;
    for (int column = expanded + (int)threadIdx.x; column < out_width; column += blockDim.x) {
      const int off = column - expanded;
      out[(int64_t)column * col_stride] =
          (off < tail_count && off < ratio - 1) ? map_token(tail_start + off) : -1;
    }
    if (count && threadIdx.x == 0) *count = min(expanded + tail_count, seq_len);
  }
};

__device__ __forceinline__ ExpandWriter make_expand_writer(const ExpandMeta& m, int row, int topk,
                                                           int32_t* out_row) {
  ExpandWriter w;
  const int req = m.token_to_req[row];
  const bool mapped = req >= 0 && req < m.num_requests;
  w.seq_len = mapped ? m.sequence_lengths[req] : 0;
  const int pos = (int)m.positions[row];
  const int p1 = pos + 1;
  w.complete = max(0, min(min(p1 / m.ratio, w.seq_len / m.ratio), topk));
  w.tail_start = (p1 / m.ratio) * m.ratio;
  w.tail_count = p1 - w.tail_start;
  w.out = out_row;
  w.count = m.store_counts ? m.counts + row : nullptr;
  w.table_row = m.physical ? m.table + (int64_t)(mapped ? req : 0) * m.table_row_stride : nullptr;
  w.col_stride = m.out_col_stride;
  w.page_size = m.page_size;
  w.table_width = m.table_width;
  w.ratio = m.ratio;
  w.out_width = m.out_width;
  w.page_div = m.page_div;
  w.physical = m.physical != 0;
  return w;
}

// --- loaders ---------------------------------------------------------------

struct DirectLoader {  // ids start + i over a contiguous score row
  const float* scores;
  int start;
  __device__ __forceinline__ uint32_t key(int i) const {
    return __builtin_bit_cast(uint32_t, scores[start + i]);
  }
  __device__ __forceinline__ int id(int i) const { return start + i; }
};

struct IndirectLoader {  // candidate list of ids into a score row
  const float* scores;
  const int32_t* ids;
  __device__ __forceinline__ uint32_t key(int i) const {
    return __builtin_bit_cast(uint32_t, scores[ids[i]]);
  }
  __device__ __forceinline__ int id(int i) const { return ids[i]; }
};

// --- block primitives ------------------------------------------------------

template <int THREADS>
__device__ __forceinline__ void block_minmax(uint32_t& lo, uint32_t& hi, SelectShared<THREADS>& sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    lo = min(lo, (uint32_t)__shfl_xor((int)lo, off, 64));
    hi = max(hi, (uint32_t)__shfl_xor((int)hi, off, 64));
  }
  if (lane == 0) {
    sh.wmin[wave] = lo;
    sh.wmax[wave] = hi;
  }
  __syncthreads();
  lo = 0xffffffffu;
  hi = 0u;
#pragma unroll
  for (int w = 0; w < THREADS / 64; ++w) {
    lo = min(lo, sh.wmin[w]);
    hi = max(hi, sh.wmax[w]);
  }
  __syncthreads();
}

// Exclusive scan of two counters over threads in thread order.
template <int THREADS>
__device__ __forceinline__ void block_scan2(int& a, int& b, SelectShared<THREADS>& sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int ia = a, ib = b;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int ta = __shfl_up(ia, off, 64);
    const int tb = __shfl_up(ib, off, 64);
    if (lane >= off) {
      ia += ta;
      ib += tb;
    }
  }
  if (lane == 63) {
    sh.wgt[wave] = ia;
    sh.weq[wave] = ib;
  }
  __syncthreads();
  int pa = 0, pb = 0;
#pragma unroll
  for (int w = 0; w < THREADS / 64; ++w) {
    if (w < wave) {
      pa += sh.wgt[w];
      pb += sh.weq[w];
    }
  }
  a = pa + ia - a;
  b = pb + ib - b;
}

// Exact top-k of `length` keys delivered by `load`; emits (rank, id) pairs in
// any order with ranks = position in ascending-id order. Requires
// length <= THREADS * ITEMS when length > topk.
template <int THREADS, int ITEMS, typename Loader, typename Writer>
__device__ void select_topk(const Loader& load, int length, int topk, const Writer& write,
                            SelectShared<THREADS>& sh) {
  const int tid = threadIdx.x;
  if (length <= topk) {
    for (int i = tid; i < topk; i += THREADS) write(i, i < length ? load.id(i) : -1);
    return;
  }
  const int base = tid * ITEMS;
  uint32_t key[ITEMS];
  uint32_t active = 0;
  uint32_t lo = 0xffffffffu, hi = 0u;
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    const bool a = base + j < length;
    key[j] = a ? load.key(base + j) : 0u;
    if (a) {
      active |= 1u << j;
      lo = min(lo, key[j]);
      hi = max(hi, key[j]);
    }
  }
  if (tid < 256) sh.hist[tid] = 0u;
  for (int b = tid + THREADS; b < 256; b += THREADS) sh.hist[b] = 0u;
  block_minmax<THREADS>(lo, hi, sh);

  const int lane = tid & 63;
  int remaining = topk;
  uint32_t cand = active;
  while (lo != hi) {
    const int high_bit = 31 - __builtin_clz(lo ^ hi);
    const int shift = high_bit > 7 ? high_bit - 7 : 0;
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      const bool a = (cand >> j) & 1u;
      const int d = (int)((key[j] >> shift) & 255u);
      const uint64_t am = __ballot(a);
      if (am == 0) continue;
      const int first = __builtin_ctzll(am);
      const int d_first = __shfl(d, first, 64);
      const uint64_t same = __ballot(a && d == d_first);
      if (same == am) {
        if (lane == first) atomicAdd(&sh.hist[d], (uint32_t)__builtin_popcountll(am));
      } else if (a) {
        atomicAdd(&sh.hist[d], 1u);
      }
    }
    __syncthreads();
    if (tid < 64) {
      // Suffix counts over 256 bins: lane owns bins 4*lane .. 4*lane+3.
      uint32_t h[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        h[i] = sh.hist[4 * lane + i];
        sh.hist[4 * lane + i] = 0u;
      }
      const int tot = (int)(h[0] + h[1] + h[2] + h[3]);
      int suf = tot;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_down(suf, off, 64);
        if (lane + off < 64) suf += t;
      }
      int above = suf - tot;  // candidates in bins above this lane's bins
#pragma unroll
      for (int i = 3; i >= 0; --i) {
        if (above < remaining && above + (int)h[i] >= remaining) {
          sh.bin = 4 * lane + i;
          sh.remaining = remaining - above;
        }
        above += (int)h[i];
      }
    }
    __syncthreads();
    const uint32_t bin = (uint32_t)sh.bin;
    remaining = sh.remaining;
    uint32_t next = 0;
    lo = 0xffffffffu;
    hi = 0u;
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      if (((cand >> j) & 1u) && ((key[j] >> shift) & 255u) == bin) {
        next |= 1u << j;
        lo = min(lo, key[j]);
        hi = max(hi, key[j]);
      }
    }
    cand = next;
    block_minmax<THREADS>(lo, hi, sh);
  }

  const uint32_t threshold = lo;
  int gt = 0, eq = 0;
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    if ((active >> j) & 1u) {
      gt += key[j] > threshold;
      eq += key[j] == threshold;
    }
  }
  block_scan2<THREADS>(gt, eq, sh);
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    if (!((active >> j) & 1u)) continue;
    if (key[j] > threshold) {
      write(gt + min(eq, remaining), load.id(base + j));
      ++gt;
    } else if (key[j] == threshold) {
      if (eq < remaining) write(gt + eq, load.id(base + j));
      ++eq;
    }
  }
}

// --- kernels ---------------------------------------------------------------

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
  int expand;
  ExpandMeta meta;
};

// Rows longer than k are scored from the logits row, so their length is
// clamped to the row width (a longer length reads past the row in the
// reference). Rows of at most k entries only emit ids and keep their length.
__device__ __forceinline__ int row_length(const TopkArgs& a, int row) {
  const int length = a.lengths[row];
  return length > a.topk ? min(length, a.cols) : length;
}

template <int THREADS, int ITEMS>
__global__ __launch_bounds__(THREADS) void topk_direct_kernel(const TopkArgs a) {
  __shared__ SelectShared<THREADS> sh;
  const int row = blockIdx.x;
  const float* srow = a.scores + (int64_t)row * a.score_row_stride;
  int32_t* orow = a.out + (int64_t)row * a.out_row_stride;
  const DirectLoader load{srow, 0};
  const int length = row_length(a, row);
  if (a.expand) {
    const ExpandWriter w = make_expand_writer(a.meta, row, a.topk, orow);
    select_topk<THREADS, ITEMS>(load, length, a.topk, w, sh);
    w.finish();
  } else {
    select_topk<THREADS, ITEMS>(load, length, a.topk, CompressedWriter{orow}, sh);
  }
}

// Pass 1 of long rows: rows short enough for one pass finish in partition 0.
template <int THREADS, int ITEMS>
__global__ __launch_bounds__(THREADS) void topk_partition_kernel(const TopkArgs a) {
  __shared__ SelectShared<THREADS> sh;
  const int row = blockIdx.x;
  const int part = blockIdx.y;
  const int length = row_length(a, row);
  const float* srow = a.scores + (int64_t)row * a.score_row_stride;
  if (length <= kPartitionColumns) {
    if (part != 0) return;
    int32_t* orow = a.out + (int64_t)row * a.out_row_stride;
    const DirectLoader load{srow, 0};
    if (a.expand) {
      const ExpandWriter w = make_expand_writer(a.meta, row, a.topk, orow);
      select_topk<THREADS, ITEMS>(load, length, a.topk, w, sh);
      w.finish();
    } else {
      select_topk<THREADS, ITEMS>(load, length, a.topk, CompressedWriter{orow}, sh);
    }
    return;
  }
  const int start = part * kPartitionColumns;
  if (start >= length) return;
  const int count = min(kPartitionColumns, length - start);
  int32_t* prow = a.partial + ((int64_t)row * a.parts + part) * a.topk;
  select_topk<THREADS, ITEMS>(DirectLoader{srow, start}, count, a.topk, CompressedWriter{prow}, sh);
}

// Pass 2: exact top-k over the concatenated partition winners (ascending ids).
template <int THREADS, int ITEMS>
__global__ __launch_bounds__(THREADS) void topk_merge_kernel(const TopkArgs a) {
  __shared__ SelectShared<THREADS> sh;
  const int row = blockIdx.x;
  const int length = row_length(a, row);
  if (length <= kPartitionColumns) return;
  const int count = (length / kPartitionColumns) * a.topk + min(length % kPartitionColumns, a.topk);
  const float* srow = a.scores + (int64_t)row * a.score_row_stride;
  int32_t* orow = a.out + (int64_t)row * a.out_row_stride;
  const IndirectLoader load{srow, a.partial + (int64_t)row * a.parts * a.topk};
  if (a.expand) {
    const ExpandWriter w = make_expand_writer(a.meta, row, a.topk, orow);
    select_topk<THREADS, ITEMS>(load, count, a.topk, w, sh);
    w.finish();
  } else {
    select_topk<THREADS, ITEMS>(load, count, a.topk, CompressedWriter{orow}, sh);
  }
}

template <int THREADS, int ITEMS>
hipError_t launch_direct(const TopkArgs& a, int rows, hipStream_t s) {
  hipLaunchKernelGGL((topk_direct_kernel<THREADS, ITEMS>), dim3(rows), dim3(THREADS), 0, s, a);
  return hipGetLastError();
}

int partitions_for(int cols) { return (cols + kPartitionColumns - 1) / kPartitionColumns; }

int launch_topk(TopkArgs a, int rows, int cols, void* workspace, size_t workspace_bytes,
                hipStream_t s) {
  if (rows == 0) return QSA_OK;
  hipError_t err;
  if (cols <= kMaxDirectColumns) {
    if (cols <= 1024) err = launch_direct<256, 4>(a, rows, s);
    else if (cols <= 2048) err = launch_direct<256, 8>(a, rows, s);
    else if (cols <= 4096) err = launch_direct<512, 8>(a, rows, s);
    else if (cols <= 8192) err = launch_direct<1024, 8>(a, rows, s);
    else err = launch_direct<1024, 16>(a, rows, s);
    if (err != hipSuccess) return fail(QSA_ERR_HIP, std::string("qsa_topk launch: ") + hipGetErrorString(err));
    return QSA_OK;
  }
  const int parts = partitions_for(cols);
  if ((int64_t)parts * a.topk > kMaxDirectColumns)
    return fail(QSA_ERR_UNSUPPORTED, "qsa_topk: partition winners exceed 16384 candidates");
  if (a.topk > kPartitionColumns)
    return fail(QSA_ERR_UNSUPPORTED, "qsa_topk: topk above 8192 with rows above 32768 columns");
  const size_t need = (size_t)rows * parts * a.topk * sizeof(int32_t);
  if (!workspace || workspace_bytes < need)
    return fail(QSA_ERR_WORKSPACE, "qsa_topk: workspace too small for partition winners");
  a.partial = static_cast<int32_t*>(workspace);
  a.parts = parts;
  hipLaunchKernelGGL((topk_partition_kernel<1024, 8>), dim3(rows, parts), dim3(1024), 0, s, a);
  if ((err = hipGetLastError()) != hipSuccess)
    return fail(QSA_ERR_HIP, std::string("qsa_topk partition launch: ") + hipGetErrorString(err));
  hipLaunchKernelGGL((topk_merge_kernel<1024, 16>), dim3(rows), dim3(1024), 0, s, a);
  if ((err = hipGetLastError()) != hipSuccess)
    return fail(QSA_ERR_HIP, std::string("qsa_topk merge launch: ") + hipGetErrorString(err));
  return QSA_OK;
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
  a.expand = 0;
  return launch_topk(a, rows, cols, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int qsa_topk_expand(const float* scores, int64_t score_row_stride, int rows, int cols,
                               const int32_t* lengths, const int64_t* positions,
                               const int32_t* sequence_lengths, int num_requests,
                               const int32_t* token_to_req, const int32_t* table,
                               int64_t table_row_stride, int table_width, int32_t* output,
                               int64_t output_row_stride, int64_t output_col_stride,
                               int output_width, int32_t* counts, int ratio, int page_size,
                               int physical, int store_counts, void* workspace,
                               size_t workspace_bytes, void* stream) {
  if (ratio <= 0) return fail(QSA_ERR_INVALID, "qsa_topk_expand: ratio must be positive");
  const int topk = output_width / ratio;
  int st = check_common(scores, rows, cols, lengths, output, topk, "qsa_topk_expand");
  if (st != QSA_OK || rows == 0) return st;
  if (!positions || !sequence_lengths || !token_to_req)
    return fail(QSA_ERR_INVALID, "qsa_topk_expand: null metadata pointer");
  if (physical && (!table || page_size <= 0))
    return fail(QSA_ERR_INVALID, "qsa_topk_expand: physical mapping needs a table and page_size");
  if (store_counts && !counts) return fail(QSA_ERR_INVALID, "qsa_topk_expand: null counts");
  TopkArgs a = {};
  a.scores = scores;
  a.score_row_stride = score_row_stride;
  a.lengths = lengths;
  a.out = output;
  a.out_row_stride = output_row_stride;
  a.topk = topk;
  a.cols = cols;
  a.expand = 1;
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
  a.meta.out_width = output_width;
  a.meta.physical = physical ? 1 : 0;
  a.meta.store_counts = store_counts ? 1 : 0;
  return launch_topk(a, rows, cols, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}
