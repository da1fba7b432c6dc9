// torch.ops.yulan_qsa_kernels: the torch-op layer over libqsa_hip.so.
//
// `topk` and `topk_expand` keep the reference plugin's schemas verbatim
// (ops/csrc/topk.cu:548-557 registers them the same way: C++ definitions
// with CUDA-key implementations); the indexer preparation, scoring, sparse
// attention and helper ops are this library's, in the same namespace.
// `select_decode` / `select_prefill` run a whole selection (scoring into a
// logits buffer, then top-k + expansion, in row spans under a memory cap),
// which is what the Python entry points of ops/indexer.py call.
//
// Every implementation checks dtypes, devices and layouts (TORCH_CHECK, a
// RuntimeError in Python, like the reference's data_ptr<T>() failures),
// takes workspaces from the caching allocator, and calls the C ABI on the
// current HIP stream of the tensors' device with that device current.
// Nothing synchronises, so every op can be captured in a HIP graph.
// Host-only code: built with the host compiler against PyTorch's headers.

#include <ATen/ATen.h>
#include <c10/hip/HIPGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <algorithm>
#include <initializer_list>
#include <optional>

#include "qsa_hip.h"

namespace {

using at::Tensor;
using OptTensor = std::optional<Tensor>;

#define QSA_REQUIRE(cond, ...) TORCH_CHECK((cond), "yulan_qsa_kernels: ", __VA_ARGS__)

void check(int status, const char* what) {
  TORCH_CHECK(status == QSA_OK, "yulan_qsa_kernels: ", what, " failed with status ", status,
              ": ", qsa_last_error());
}

const Tensor* opt(const OptTensor& t) { return t.has_value() ? &*t : nullptr; }

// The one GPU every given tensor is on.
c10::Device on_gpu(std::initializer_list<const Tensor*> tensors) {
  std::optional<c10::Device> dev;
  for (const Tensor* t : tensors) {
    if (!t) continue;
    QSA_REQUIRE(t->is_cuda(), "expected a GPU tensor, got device ", t->device());
    if (!dev) dev = t->device();
    QSA_REQUIRE(t->device() == *dev, "all tensors must be on the same device");
  }
  QSA_REQUIRE(dev.has_value(), "no tensor given");
  return *dev;
}

hipStream_t stream_of(const c10::Device& dev) {
  return c10::hip::getCurrentHIPStream(dev.index()).stream();
}

// Stride of dim d, 0 for a size-1 dim (never used to address memory; views
// may carry any value there).
int64_t sdim(const Tensor& t, int64_t d) { return t.size(d) == 1 ? 0 : t.stride(d); }

void dtype(const Tensor& t, at::ScalarType s, const char* name) {
  QSA_REQUIRE(t.scalar_type() == s, name, " must be ", s, ", got ", t.scalar_type());
}

void vec(const Tensor& t, at::ScalarType s, const char* name, int64_t min_len = -1) {
  dtype(t, s, name);
  QSA_REQUIRE(t.dim() == 1, name, " must be 1-D");
  QSA_REQUIRE(t.numel() <= 1 || t.stride(0) == 1, name, " must be contiguous");
  if (min_len >= 0)
    QSA_REQUIRE(t.numel() >= min_len, name, " has ", t.numel(), " entries, need ", min_len);
}

void positions(const Tensor& t, int64_t n, const char* name) {
  dtype(t, at::kLong, name);
  QSA_REQUIRE(t.dim() == 1 && t.numel() >= n, name, " must be 1-D with at least ", n, " entries");
  QSA_REQUIRE(t.numel() <= 1 || t.stride(0) == 1, name, " must be contiguous");
}

void unit_dim(const Tensor& t, const char* name, int64_t dims) {
  dtype(t, at::kBFloat16, name);
  QSA_REQUIRE(t.dim() == dims && t.stride(-1) == 1, name, " must be ", dims,
              "-D with unit dim stride");
}

void bf16_vec(const Tensor& t, int64_t n, const char* name) {
  dtype(t, at::kBFloat16, name);
  QSA_REQUIRE(t.dim() == 1 && t.numel() == n && (n <= 1 || t.stride(0) == 1), name,
              " must be a contiguous [", n, "] vector");
}

void rotary_table(const Tensor& cos_sin, int64_t rotary_dim) {
  dtype(cos_sin, at::kBFloat16, "cos_sin");
  QSA_REQUIRE(cos_sin.dim() == 2 && cos_sin.size(1) == rotary_dim && cos_sin.is_contiguous(),
              "cos_sin must be a contiguous [positions, rotary_dim] tensor");
}

void table2d(const Tensor& t, const char* name) {
  dtype(t, at::kInt, name);
  QSA_REQUIRE(t.dim() == 2 && (t.size(1) <= 1 || t.stride(1) == 1), name,
              " must be [requests, width] with unit column stride");
}

void scores2d(const Tensor& t, const char* name) {
  dtype(t, at::kFloat, name);
  QSA_REQUIRE(t.dim() == 2 && (t.size(1) <= 1 || t.stride(1) == 1), name,
              " must be [rows, cols] with unit column stride");
}

Tensor workspace(size_t bytes, const c10::Device& dev) {
  return at::empty({(int64_t)std::max<size_t>(bytes, 1)},
                   at::TensorOptions().dtype(at::kByte).device(dev));
}

// Typed pointer to element `offset` of t's storage view (elements of T).
template <typename T>
T* at_elem(const Tensor& t, int64_t offset = 0) {
  return static_cast<T*>(t.data_ptr()) + offset;
}

const void* ptr_or_null(const Tensor* t) { return t ? t->data_ptr() : nullptr; }

// --- topk / topk_expand (reference schemas) ---------------------------------

void topk_impl(const Tensor& scores, const Tensor& lengths, const Tensor& output) {
  const auto dev = on_gpu({&scores, &lengths, &output});
  scores2d(scores, "scores");
  vec(lengths, at::kInt, "lengths", scores.size(0));
  dtype(output, at::kInt, "output");
  QSA_REQUIRE(output.dim() == 2 && output.size(0) == scores.size(0) &&
                  (output.size(1) <= 1 || output.stride(1) == 1),
              "output must be [rows, topk] with unit column stride");
  const int rows = (int)scores.size(0), cols = (int)scores.size(1);
  if (rows == 0) return;
  const int topk = (int)output.size(1);
  c10::hip::HIPGuard guard(dev.index());
  const size_t ws_bytes = qsa_topk_workspace_bytes(rows, cols, topk);
  Tensor ws = ws_bytes ? workspace(ws_bytes, dev) : Tensor();
  check(qsa_topk(at_elem<float>(scores), scores.stride(0), rows, cols, at_elem<int32_t>(lengths),
                 at_elem<int32_t>(output), output.stride(0), topk,
                 ws_bytes ? ws.data_ptr() : nullptr, ws_bytes, stream_of(dev)),
        "qsa_topk");
}

struct ExpandArgs {
  const Tensor* table;  // null unless physical
  const Tensor* counts;  // null unless store_counts
  int64_t ratio, page_size;
};

void check_expand(const Tensor& positions_t, const Tensor& sequence_lengths,
                  const Tensor& token_to_req, const Tensor& output, int64_t rows,
                  const ExpandArgs& e) {
  vec(positions_t, at::kLong, "positions", rows);
  vec(sequence_lengths, at::kInt, "sequence_lengths");
  vec(token_to_req, at::kInt, "token_to_req", rows);
  dtype(output, at::kInt, "output");
  QSA_REQUIRE(output.dim() == 2 && output.size(0) >= rows, "output must be [rows, width]");
  QSA_REQUIRE(e.ratio > 0, "ratio must be positive");
  if (e.table) {
    table2d(*e.table, "table");
    QSA_REQUIRE(e.page_size > 0, "page_size must be positive");
  }
  if (e.counts) vec(*e.counts, at::kInt, "counts", rows);
}

// qsa_topk_expand over rows [r0, r0 + rows) of the caller's row tensors with
// logits rows from `scores` (its own row 0 = caller row r0).
void launch_expand(const Tensor& scores, int rows, const Tensor& lengths, const Tensor& pos,
                   const Tensor& sequence_lengths, const Tensor& token_to_req,
                   const Tensor& output, const ExpandArgs& e, int64_t r0,
                   const c10::Device& dev, hipStream_t s) {
  const int cols = (int)scores.size(1);
  const int width = (int)output.size(1);
  const int topk = width / (int)e.ratio;
  const size_t ws_bytes = qsa_topk_workspace_bytes(rows, cols, topk);
  Tensor ws = ws_bytes ? workspace(ws_bytes, dev) : Tensor();
  check(qsa_topk_expand(
            at_elem<float>(scores), scores.stride(0), rows, cols, at_elem<int32_t>(lengths, r0),
            at_elem<int64_t>(pos, r0), at_elem<int32_t>(sequence_lengths),
            (int)sequence_lengths.numel(), at_elem<int32_t>(token_to_req, r0),
            e.table ? at_elem<int32_t>(*e.table) : nullptr, e.table ? e.table->stride(0) : 0,
            e.table ? (int)e.table->size(1) : 0, at_elem<int32_t>(output, r0 * output.stride(0)),
            output.stride(0), output.stride(1), width,
            e.counts ? at_elem<int32_t>(*e.counts, r0) : nullptr, (int)e.ratio,
            (int)e.page_size, e.table ? 1 : 0, e.counts ? 1 : 0,
            ws_bytes ? ws.data_ptr() : nullptr, ws_bytes, s),
        "qsa_topk_expand");
}

void topk_expand_impl(const Tensor& scores, const Tensor& lengths, const Tensor& pos,
                      const Tensor& sequence_lengths, const Tensor& token_to_req,
                      const Tensor& table, const Tensor& output, const Tensor& counts,
                      int64_t ratio, int64_t page_size, bool physical, bool store_counts) {
  const auto dev =
      on_gpu({&scores, &lengths, &pos, &sequence_lengths, &token_to_req, &table, &output, &counts});
  scores2d(scores, "scores");
  const int64_t rows = scores.size(0);
  vec(lengths, at::kInt, "lengths", rows);
  const ExpandArgs e{physical ? &table : nullptr, store_counts ? &counts : nullptr, ratio,
                     page_size};
  check_expand(pos, sequence_lengths, token_to_req, output, rows, e);
  QSA_REQUIRE(output.size(0) == rows, "output must be [rows, width]");
  if (rows == 0) return;
  c10::hip::HIPGuard guard(dev.index());
  launch_expand(scores, (int)rows, lengths, pos, sequence_lengths, token_to_req, output, e, 0,
                dev, stream_of(dev));
}

// --- indexer scoring ----------------------------------------------------------

struct CacheView {
  int64_t block_stride, token_stride;
};

CacheView index_cache(const Tensor& k_cache, int64_t dim) {
  dtype(k_cache, at::kBFloat16, "k_cache");
  QSA_REQUIRE(k_cache.dim() == 3 || k_cache.dim() == 4, "k_cache must be [blocks, page, (1,) dim]");
  if (k_cache.dim() == 4) QSA_REQUIRE(k_cache.size(2) == 1, "k_cache must hold one index head");
  QSA_REQUIRE(k_cache.stride(-1) == 1, "k_cache must have a unit dim stride");
  QSA_REQUIRE(k_cache.size(-1) == dim, "k_cache dim must match q");
  return {sdim(k_cache, 0), sdim(k_cache, 1)};
}

void check_index_q(const Tensor& q) {
  dtype(q, at::kBFloat16, "q");
  QSA_REQUIRE(q.dim() == 3 && q.stride(2) == 1, "q must be [rows, heads, dim] with unit dim stride");
}

void indexer_decode_impl(const Tensor& q, const Tensor& k_cache, const Tensor& page_table,
                         const Tensor& visible, const Tensor& logits, int64_t decode_query_len) {
  const auto dev = on_gpu({&q, &k_cache, &page_table, &visible, &logits});
  check_index_q(q);
  const int64_t rows = q.size(0);
  const CacheView c = index_cache(k_cache, q.size(2));
  table2d(page_table, "page_table");
  vec(visible, at::kInt, "visible", rows);
  scores2d(logits, "logits");
  QSA_REQUIRE(logits.size(0) >= rows, "logits has fewer rows than q");
  QSA_REQUIRE(decode_query_len > 0 && page_table.size(0) * decode_query_len >= rows,
              "page_table has fewer requests than rows / decode_query_len");
  if (rows == 0) return;
  c10::hip::HIPGuard guard(dev.index());
  check(qsa_indexer_decode(q.data_ptr(), sdim(q, 0), sdim(q, 1), (int)rows, (int)q.size(1),
                           (int)q.size(2), k_cache.data_ptr(), c.block_stride, c.token_stride,
                           (int)k_cache.size(0), (int)k_cache.size(1),
                           at_elem<int32_t>(page_table), page_table.stride(0),
                           (int)page_table.size(1), at_elem<int32_t>(visible),
                           (int)decode_query_len, at_elem<float>(logits), logits.stride(0),
                           (int)logits.size(1), stream_of(dev)),
        "qsa_indexer_decode");
}

void check_prefill(const Tensor& q, const Tensor& page_table, const Tensor& query_start_loc,
                   const Tensor& visible, int64_t query_offset, int64_t num_rows) {
  check_index_q(q);
  table2d(page_table, "page_table");
  vec(query_start_loc, at::kInt, "query_start_loc", page_table.size(0) + 1);
  vec(visible, at::kInt, "visible", query_offset + num_rows);
  QSA_REQUIRE(query_offset >= 0 && q.size(0) >= query_offset + num_rows,
              "q has fewer rows than query_offset + num_rows");
}

int prefill_launch(const Tensor& q, const Tensor& k_cache, const CacheView& c,
                   const Tensor& page_table, const Tensor& query_start_loc, const Tensor& visible,
                   const Tensor& logits, int64_t query_offset, int64_t num_rows,
                   int64_t max_query_len, hipStream_t s) {
  return qsa_indexer_prefill(q.data_ptr(), sdim(q, 0), sdim(q, 1), (int)q.size(1),
                             (int)q.size(2), k_cache.data_ptr(), c.block_stride, c.token_stride,
                             (int)k_cache.size(0), (int)k_cache.size(1),
                             at_elem<int32_t>(page_table), page_table.stride(0),
                             (int)page_table.size(1), (int)page_table.size(0),
                             at_elem<int32_t>(query_start_loc), at_elem<int32_t>(visible),
                             (int)query_offset, (int)num_rows, (int)max_query_len,
                             at_elem<float>(logits), logits.stride(0), (int)logits.size(1), s);
}

void indexer_prefill_impl(const Tensor& q, const Tensor& k_cache, const Tensor& page_table,
                          const Tensor& query_start_loc, const Tensor& visible,
                          const Tensor& logits, int64_t query_offset, int64_t num_rows,
                          int64_t max_query_len) {
  const auto dev = on_gpu({&q, &k_cache, &page_table, &query_start_loc, &visible, &logits});
  check_prefill(q, page_table, query_start_loc, visible, query_offset, num_rows);
  const CacheView c = index_cache(k_cache, q.size(2));
  scores2d(logits, "logits");
  QSA_REQUIRE(logits.size(0) >= num_rows, "logits has fewer rows than num_rows");
  if (num_rows == 0 || page_table.size(0) == 0) return;
  c10::hip::HIPGuard guard(dev.index());
  check(prefill_launch(q, k_cache, c, page_table, query_start_loc, visible, logits, query_offset,
                       num_rows, max_query_len, stream_of(dev)),
        "qsa_indexer_prefill");
}

// --- whole selections (ops/indexer.py:227-343) ---------------------------------

// Decode: request i of page_table owns rows [i * dql, (i + 1) * dql). Scores
// into a [rows, columns] fp32 buffer of at most cap_bytes (whole requests per
// span), then top-k + expansion of each span.
void select_decode_impl(const Tensor& q, const Tensor& k_cache, const Tensor& page_table,
                        const Tensor& visible, const Tensor& pos, const Tensor& sequence_lengths,
                        const Tensor& token_to_req, const Tensor& output, const OptTensor& table,
                        const OptTensor& counts, int64_t ratio, int64_t decode_query_len,
                        int64_t columns, int64_t page_size, int64_t cap_bytes) {
  const auto dev = on_gpu({&q, &k_cache, &page_table, &visible, &pos, &sequence_lengths,
                           &token_to_req, &output, opt(table), opt(counts)});
  check_index_q(q);
  const int64_t rows = q.size(0);
  const CacheView c = index_cache(k_cache, q.size(2));
  table2d(page_table, "page_table");
  vec(visible, at::kInt, "visible", rows);
  const ExpandArgs e{opt(table), opt(counts), ratio, page_size};
  check_expand(pos, sequence_lengths, token_to_req, output, rows, e);
  QSA_REQUIRE(decode_query_len > 0 && rows % decode_query_len == 0 &&
                  page_table.size(0) * decode_query_len >= rows,
              "rows must be whole requests of decode_query_len rows of page_table");
  QSA_REQUIRE(columns > 0, "columns must be positive");
  if (rows == 0) return;
  const int64_t dql = decode_query_len;
  const int64_t requests = rows / dql;
  const int64_t per_span = std::max<int64_t>(1, cap_bytes / (4 * columns * dql));
  c10::hip::HIPGuard guard(dev.index());
  const hipStream_t s = stream_of(dev);
  Tensor logits = at::empty({std::min(requests, per_span) * dql, columns},
                            at::TensorOptions().dtype(at::kFloat).device(dev));
  for (int64_t r0 = 0; r0 < requests; r0 += per_span) {
    const int64_t r1 = std::min(requests, r0 + per_span);
    const int64_t row0 = r0 * dql, n = (r1 - r0) * dql;
    check(qsa_indexer_decode(static_cast<char*>(q.data_ptr()) + row0 * q.stride(0) * 2,
                             sdim(q, 0), sdim(q, 1), (int)n, (int)q.size(1), (int)q.size(2),
                             k_cache.data_ptr(), c.block_stride, c.token_stride,
                             (int)k_cache.size(0), (int)k_cache.size(1),
                             at_elem<int32_t>(page_table, r0 * page_table.stride(0)),
                             page_table.stride(0), (int)page_table.size(1),
                             at_elem<int32_t>(visible, row0), (int)dql, at_elem<float>(logits),
                             logits.stride(0), (int)logits.size(1), s),
          "qsa_indexer_decode");
    launch_expand(logits.narrow(0, 0, n), (int)n, visible, pos, sequence_lengths, token_to_req,
                  output, e, row0, dev, s);
  }
}

// Prefill: the rows of q are the packed query tokens of page_table's
// requests (request i from row query_start_loc[i] - query_start_loc[0]).
// Scores in row spans of at most cap_bytes of fp32 logits of `width`
// columns (rounded to whole launch rounds by the library), then top-k +
// expansion of each span.
void select_prefill_impl(const Tensor& q, const Tensor& k_cache, const Tensor& page_table,
                         const Tensor& query_start_loc, const Tensor& visible, const Tensor& pos,
                         const Tensor& sequence_lengths, const Tensor& token_to_req,
                         const Tensor& output, const OptTensor& table, const OptTensor& counts,
                         int64_t ratio, int64_t max_query_len, int64_t width, int64_t page_size,
                         int64_t cap_bytes) {
  const auto dev = on_gpu({&q, &k_cache, &page_table, &query_start_loc, &visible, &pos,
                           &sequence_lengths, &token_to_req, &output, opt(table), opt(counts)});
  const int64_t rows = q.size(0);
  check_prefill(q, page_table, query_start_loc, visible, 0, rows);
  const CacheView c = index_cache(k_cache, q.size(2));
  const ExpandArgs e{opt(table), opt(counts), ratio, page_size};
  check_expand(pos, sequence_lengths, token_to_req, output, rows, e);
  QSA_REQUIRE(width > 0, "width must be positive");
  if (rows == 0) return;
  const int64_t per_span =
      std::max<int64_t>(1, qsa_indexer_prefill_span_rows((int)width, cap_bytes));
  c10::hip::HIPGuard guard(dev.index());
  const hipStream_t s = stream_of(dev);
  Tensor logits = at::empty({std::min(rows, per_span), width},
                            at::TensorOptions().dtype(at::kFloat).device(dev));
  for (int64_t a = 0; a < rows; a += per_span) {
    const int64_t n = std::min(rows, a + per_span) - a;
    if (page_table.size(0) > 0)
      check(prefill_launch(q, k_cache, c, page_table, query_start_loc, visible, logits, a, n,
                           max_query_len, s),
            "qsa_indexer_prefill");
    launch_expand(logits.narrow(0, 0, n), (int)n, visible, pos, sequence_lengths, token_to_req,
                  output, e, a, dev, s);
  }
}

// --- sparse attention -----------------------------------------------------------

struct GateStrides {
  int64_t row = 0, head = 0, dim = 0;
};

GateStrides gate_strides(const OptTensor& gate, int64_t rows, int64_t heads, int64_t dim) {
  if (!gate) return {};
  dtype(*gate, at::kBFloat16, "output_gate");
  QSA_REQUIRE(gate->dim() == 3 && gate->size(1) == heads && gate->size(2) == dim &&
                  gate->size(0) >= rows,
              "output_gate must be [rows, heads, dim]");
  return {sdim(*gate, 0), sdim(*gate, 1), sdim(*gate, 2)};
}

void check_out(const Tensor& out, int64_t rows, int64_t heads, int64_t dim) {
  dtype(out, at::kBFloat16, "out");
  QSA_REQUIRE(out.dim() == 3 && out.size(1) == heads && out.size(2) == dim &&
                  out.size(0) >= rows && out.stride(2) == 1,
              "out must be [rows, heads, dim] with unit dim stride");
}

// num_splits <= 0: the library's choice for this shape (decode launch shapes
// when the indices are physical slots).
void sparse_attention_impl(const Tensor& q, const Tensor& k_cache, const Tensor& v_cache,
                           const Tensor& indices, const Tensor& block_table,
                           const Tensor& token_to_req, const Tensor& out,
                           const OptTensor& output_gate, const OptTensor& valid_counts,
                           bool indices_are_physical, int64_t num_splits) {
  const auto dev = on_gpu({&q, &k_cache, &v_cache, &indices, &block_table, &token_to_req, &out,
                           opt(output_gate), opt(valid_counts)});
  dtype(q, at::kBFloat16, "q");
  dtype(k_cache, at::kBFloat16, "k_cache");
  dtype(v_cache, at::kBFloat16, "v_cache");
  QSA_REQUIRE(q.dim() == 3 && q.stride(2) == 1, "q must be [rows, heads, dim] with unit dim stride");
  const int64_t rows = q.size(0), hq = q.size(1), dim = q.size(2);
  QSA_REQUIRE(k_cache.dim() == 4 && v_cache.dim() == 4 && k_cache.sizes() == v_cache.sizes(),
              "k_cache/v_cache must be [blocks, page, kv_heads, dim] of one shape");
  QSA_REQUIRE(k_cache.stride(3) == 1 && v_cache.stride(3) == 1, "k/v caches need a unit dim stride");
  QSA_REQUIRE(k_cache.size(3) == dim, "cache head dim must match q");
  check_out(out, rows, hq, dim);
  dtype(indices, at::kInt, "indices");
  QSA_REQUIRE(indices.dim() == 2 && indices.size(0) >= rows &&
                  (indices.size(1) <= 1 || indices.stride(1) == 1),
              "indices must be [rows, width] with unit column stride");
  table2d(block_table, "block_table");
  vec(token_to_req, at::kInt, "token_to_req", rows);
  if (valid_counts) vec(*valid_counts, at::kInt, "valid_counts", rows);
  const GateStrides g = gate_strides(output_gate, rows, hq, dim);
  if (rows == 0) return;
  c10::hip::HIPGuard guard(dev.index());
  int splits = (int)num_splits;
  if (splits <= 0)
    splits = qsa_sparse_attention_splits((int)rows, (int)hq, (int)k_cache.size(2), (int)dim,
                                         (int)indices.size(1), indices_are_physical ? 1 : 0);
  const size_t ws_bytes = qsa_sparse_attention_workspace_bytes((int)rows, (int)hq, (int)dim, splits);
  Tensor ws = ws_bytes ? workspace(ws_bytes, dev) : Tensor();
  check(qsa_sparse_attention(
            q.data_ptr(), sdim(q, 0), sdim(q, 1), (int)rows, (int)hq, (int)dim,
            k_cache.data_ptr(), sdim(k_cache, 0), sdim(k_cache, 1), sdim(k_cache, 2),
            v_cache.data_ptr(), sdim(v_cache, 0), sdim(v_cache, 1), sdim(v_cache, 2),
            (int)k_cache.size(0), (int)k_cache.size(1), (int)k_cache.size(2),
            at_elem<int32_t>(indices), indices.stride(0), (int)indices.size(1),
            at_elem<int32_t>(block_table), block_table.stride(0), (int)block_table.size(1),
            (int)block_table.size(0), at_elem<int32_t>(token_to_req),
            valid_counts ? at_elem<int32_t>(*valid_counts) : nullptr, out.data_ptr(),
            sdim(out, 0), sdim(out, 1), ptr_or_null(opt(output_gate)), g.row, g.head, g.dim,
            indices_are_physical ? 1 : 0, splits, ws_bytes ? ws.data_ptr() : nullptr, ws_bytes,
            stream_of(dev)),
        "qsa_sparse_attention");
}

// Decode rows: top-k + physical expansion of `scores` into indices/counts,
// then the sparse attention over them (qsa_decode_select_attention: one
// launch for the shapes it fuses). The expansion's page size is the main
// cache's.
void decode_select_attend_impl(const Tensor& scores, const Tensor& lengths, const Tensor& pos,
                               const Tensor& sequence_lengths, const Tensor& token_to_req,
                               const Tensor& table, const Tensor& indices, const Tensor& counts,
                               int64_t ratio, const Tensor& q, const Tensor& k_cache,
                               const Tensor& v_cache, const Tensor& out,
                               const OptTensor& output_gate, int64_t num_splits) {
  const auto dev = on_gpu({&scores, &lengths, &pos, &sequence_lengths, &token_to_req, &table,
                           &indices, &counts, &q, &k_cache, &v_cache, &out, opt(output_gate)});
  scores2d(scores, "scores");
  const int64_t rows = scores.size(0);
  vec(lengths, at::kInt, "lengths", rows);
  QSA_REQUIRE(k_cache.dim() == 4, "k_cache must be [blocks, page, kv_heads, dim]");
  const ExpandArgs e{&table, &counts, ratio, k_cache.size(1)};
  check_expand(pos, sequence_lengths, token_to_req, indices, rows, e);
  QSA_REQUIRE(indices.size(0) == rows && indices.stride(1) == 1,
              "indices must be [rows, width] with unit column stride");
  dtype(q, at::kBFloat16, "q");
  dtype(k_cache, at::kBFloat16, "k_cache");
  dtype(v_cache, at::kBFloat16, "v_cache");
  QSA_REQUIRE(q.dim() == 3 && q.stride(2) == 1 && q.size(0) == rows,
              "q must be [rows, heads, dim] with unit dim stride");
  const int64_t hq = q.size(1), dim = q.size(2);
  QSA_REQUIRE(v_cache.dim() == 4 && k_cache.sizes() == v_cache.sizes(),
              "k_cache/v_cache must be [blocks, page, kv_heads, dim] of one shape");
  QSA_REQUIRE(k_cache.stride(3) == 1 && v_cache.stride(3) == 1, "k/v caches need a unit dim stride");
  QSA_REQUIRE(k_cache.size(3) == dim, "cache head dim must match q");
  check_out(out, rows, hq, dim);
  const GateStrides g = gate_strides(output_gate, rows, hq, dim);
  if (rows == 0) return;
  c10::hip::HIPGuard guard(dev.index());
  const int cols = (int)scores.size(1), width = (int)indices.size(1);
  int splits = (int)num_splits;
  if (splits <= 0)
    splits = qsa_sparse_attention_splits((int)rows, (int)hq, (int)k_cache.size(2), (int)dim,
                                         width, 1);
  const size_t ws_bytes = qsa_decode_select_attention_workspace_bytes(
      (int)rows, cols, width, (int)ratio, (int)hq, (int)dim, splits);
  Tensor ws = ws_bytes ? workspace(ws_bytes, dev) : Tensor();
  check(qsa_decode_select_attention(
            at_elem<float>(scores), scores.stride(0), (int)rows, cols, at_elem<int32_t>(lengths),
            at_elem<int64_t>(pos), at_elem<int32_t>(sequence_lengths),
            (int)sequence_lengths.numel(), at_elem<int32_t>(token_to_req), at_elem<int32_t>(table),
            table.stride(0), (int)table.size(1), (int)ratio, at_elem<int32_t>(indices),
            indices.stride(0), width, at_elem<int32_t>(counts), q.data_ptr(), sdim(q, 0),
            sdim(q, 1), (int)hq, (int)dim, k_cache.data_ptr(), sdim(k_cache, 0),
            sdim(k_cache, 1), sdim(k_cache, 2), v_cache.data_ptr(), sdim(v_cache, 0),
            sdim(v_cache, 1), sdim(v_cache, 2), (int)k_cache.size(0), (int)k_cache.size(1),
            (int)k_cache.size(2), out.data_ptr(), sdim(out, 0), sdim(out, 1),
            ptr_or_null(opt(output_gate)), g.row, g.head, g.dim, splits,
            ws_bytes ? ws.data_ptr() : nullptr, ws_bytes, stream_of(dev)),
        "qsa_decode_select_attention");
}

void sparse_attention_merge_impl(const Tensor& partial_out, const Tensor& partial_lse,
                                 const Tensor& out, const OptTensor& output_gate) {
  const auto dev = on_gpu({&partial_out, &partial_lse, &out, opt(output_gate)});
  dtype(partial_out, at::kFloat, "partial_out");
  dtype(partial_lse, at::kFloat, "partial_lse");
  QSA_REQUIRE(partial_out.dim() == 4 && partial_out.is_contiguous(),
              "partial_out must be contiguous [splits, rows, heads, dim]");
  const int64_t splits = partial_out.size(0), rows = partial_out.size(1),
                hq = partial_out.size(2), dim = partial_out.size(3);
  QSA_REQUIRE(partial_lse.dim() == 3 && partial_lse.size(0) == splits &&
                  partial_lse.size(1) == rows && partial_lse.size(2) == hq &&
                  partial_lse.is_contiguous(),
              "partial_lse must be contiguous [splits, rows, heads]");
  check_out(out, rows, hq, dim);
  const GateStrides g = gate_strides(output_gate, rows, hq, dim);
  if (rows == 0) return;
  c10::hip::HIPGuard guard(dev.index());
  check(qsa_sparse_attention_merge(at_elem<float>(partial_out), at_elem<float>(partial_lse),
                                   (int)splits, (int)rows, (int)hq, (int)dim, out.data_ptr(),
                                   sdim(out, 0), sdim(out, 1),
                                   ptr_or_null(opt(output_gate)), g.row, g.head, g.dim,
                                   stream_of(dev)),
        "qsa_sparse_attention_merge");
}

// --- indexer preparation and cache helpers -------------------------------------

void indexer_prepare_impl(const Tensor& index_qk, const Tensor& pos, const Tensor& q_norm_weight,
                          const Tensor& k_norm_weight, const Tensor& cos_sin, double eps,
                          const Tensor& index_q_out, const Tensor& state_cache,
                          const Tensor& state_slots, const Tensor& state_table,
                          const Tensor& query_start_loc, const Tensor& logical_positions,
                          const Tensor& compressed_cache, const Tensor& compressed_slots,
                          const Tensor& k_work, const Tensor& main_key, const Tensor& main_value,
                          const Tensor& main_key_cache, const Tensor& main_value_cache,
                          const Tensor& main_slots, int64_t num_index_heads,
                          int64_t index_head_dim, int64_t rotary_dim, int64_t compress_ratio) {
  const auto dev = on_gpu({&index_qk, &pos, &q_norm_weight, &k_norm_weight, &cos_sin,
                           &index_q_out, &state_cache, &state_slots, &state_table,
                           &query_start_loc, &logical_positions, &compressed_cache,
                           &compressed_slots, &k_work, &main_key, &main_value, &main_key_cache,
                           &main_value_cache, &main_slots});
  const int64_t tokens = index_qk.size(0), heads = num_index_heads, dim = index_head_dim;
  unit_dim(index_qk, "index_qk", 2);
  QSA_REQUIRE(index_qk.size(1) >= (heads + 1) * dim, "index_qk must hold (heads + 1) * dim columns");
  positions(pos, tokens, "positions");
  bf16_vec(q_norm_weight, dim, "q_norm_weight");
  bf16_vec(k_norm_weight, dim, "k_norm_weight");
  rotary_table(cos_sin, rotary_dim);
  dtype(index_q_out, at::kBFloat16, "index_q_out");
  QSA_REQUIRE(index_q_out.is_contiguous() && index_q_out.numel() == tokens * heads * dim,
              "index_q_out must be a contiguous [tokens, heads, dim] tensor");
  for (auto [t, name] : {std::pair<const Tensor*, const char*>{&state_cache, "state_cache"},
                         {&compressed_cache, "compressed_cache"}}) {
    dtype(*t, at::kBFloat16, name);
    QSA_REQUIRE((t->dim() == 3 || t->dim() == 4) && t->stride(-1) == 1 && t->size(-1) == dim &&
                    (t->dim() == 3 || t->size(2) == 1),
                name, " must be [blocks, page, (1,) dim] with unit dim stride");
  }
  for (auto [t, name] : {std::pair<const Tensor*, const char*>{&state_slots, "state_slots"},
                         {&compressed_slots, "compressed_slots"},
                         {&main_slots, "main_slots"},
                         {&logical_positions, "logical_positions"}}) {
    positions(*t, tokens, name);
    QSA_REQUIRE(t->numel() <= 1 || t->stride(0) == 1, name, " must be contiguous");
  }
  dtype(state_table, at::kInt, "state_table");
  QSA_REQUIRE(state_table.dim() == 2, "state_table must be [requests, width]");
  vec(query_start_loc, at::kInt, "query_start_loc");
  const int64_t num_requests = query_start_loc.numel() - 1;
  QSA_REQUIRE(state_table.size(0) >= num_requests, "state_table has fewer rows than requests");
  dtype(k_work, at::kInt, "k_work");
  QSA_REQUIRE(k_work.dim() == 2 && k_work.size(1) == 2 && k_work.is_contiguous(),
              "k_work must be a contiguous [items, 2] tensor");
  unit_dim(main_key, "main_key", 3);
  unit_dim(main_value, "main_value", 3);
  unit_dim(main_key_cache, "main_key_cache", 4);
  unit_dim(main_value_cache, "main_value_cache", 4);
  const int64_t kv_heads = main_key.size(1), main_dim = main_key.size(2);
  QSA_REQUIRE(main_key.size(0) == tokens && main_value.size(0) == tokens &&
                  main_value.size(1) == kv_heads && main_value.size(2) == main_dim,
              "main_key / main_value must be [tokens, kv_heads, dim]");
  QSA_REQUIRE(main_key_cache.sizes() == main_value_cache.sizes() &&
                  main_key_cache.size(2) == kv_heads && main_key_cache.size(3) == main_dim,
              "main caches must be [blocks, page, kv_heads, dim] matching main_key");
  if (tokens == 0 && k_work.size(0) == 0) return;
  c10::hip::HIPGuard guard(dev.index());
  check(qsa_indexer_prepare(
            index_qk.data_ptr(), sdim(index_qk, 0), (int)tokens, at_elem<int64_t>(pos),
            sdim(pos, 0), q_norm_weight.data_ptr(), k_norm_weight.data_ptr(),
            cos_sin.data_ptr(), (int)cos_sin.size(0), (float)eps, index_q_out.data_ptr(),
            state_cache.data_ptr(), sdim(state_cache, 0), sdim(state_cache, 1),
            (int)state_cache.size(1), (int)state_cache.size(0), at_elem<int64_t>(state_slots),
            at_elem<int32_t>(state_table), sdim(state_table, 0),
            at_elem<int32_t>(query_start_loc), at_elem<int64_t>(logical_positions),
            (int)num_requests, compressed_cache.data_ptr(), sdim(compressed_cache, 0),
            sdim(compressed_cache, 1), (int)compressed_cache.size(1),
            (int)compressed_cache.size(0), at_elem<int64_t>(compressed_slots),
            at_elem<int32_t>(k_work), (int)k_work.size(0), main_key.data_ptr(),
            sdim(main_key, 0), sdim(main_key, 1), main_value.data_ptr(),
            sdim(main_value, 0), sdim(main_value, 1), main_key_cache.data_ptr(),
            sdim(main_key_cache, 0), sdim(main_key_cache, 1), sdim(main_key_cache, 2),
            main_value_cache.data_ptr(), sdim(main_value_cache, 0),
            sdim(main_value_cache, 1), sdim(main_value_cache, 2),
            at_elem<int64_t>(main_slots), (int)main_key_cache.size(1),
            (int)main_key_cache.size(0), (int)heads, (int)dim, (int)rotary_dim,
            (int)compress_ratio, (int)kv_heads, (int)main_dim, stream_of(dev)),
        "qsa_indexer_prepare");
}

void indexer_norm_rope_impl(const Tensor& values, const Tensor& weight, const Tensor& pos,
                            const Tensor& cos_sin, double eps, int64_t rotary_dim,
                            const Tensor& out) {
  const auto dev = on_gpu({&values, &weight, &pos, &cos_sin, &out});
  unit_dim(values, "values", 3);
  const int64_t tokens = values.size(0), heads = values.size(1), dim = values.size(2);
  bf16_vec(weight, dim, "weight");
  positions(pos, tokens, "positions");
  rotary_table(cos_sin, rotary_dim);
  dtype(out, at::kBFloat16, "out");
  QSA_REQUIRE(out.is_contiguous() && out.sizes() == values.sizes(),
              "out must be a contiguous tensor shaped like values");
  if (tokens == 0 || heads == 0) return;
  c10::hip::HIPGuard guard(dev.index());
  check(qsa_indexer_norm_rope(values.data_ptr(), sdim(values, 0), sdim(values, 1), (int)tokens,
                              (int)heads, (int)dim, weight.data_ptr(), at_elem<int64_t>(pos),
                              sdim(pos, 0), cos_sin.data_ptr(), (int)cos_sin.size(0),
                              (float)eps, (int)rotary_dim, out.data_ptr(), stream_of(dev)),
        "qsa_indexer_norm_rope");
}

void store_cache_rows_impl(const Tensor& cache, const Tensor& slot_mapping,
                           const Tensor& rows_in) {
  const auto dev = on_gpu({&cache, &slot_mapping, &rows_in});
  dtype(cache, at::kBFloat16, "cache");
  QSA_REQUIRE(cache.dim() == 4 && cache.stride(3) == 1,
              "cache must be [blocks, page, heads, width] with unit width stride");
  const Tensor rows = rows_in.dim() == 3 ? rows_in.select(1, 0) : rows_in;
  dtype(rows, at::kBFloat16, "rows");
  QSA_REQUIRE(rows.dim() == 2 && rows.stride(1) == 1 && rows.size(1) >= cache.size(3),
              "rows must be [rows, >= width] with unit dim stride");
  positions(slot_mapping, rows.size(0), "slot_mapping");
  QSA_REQUIRE(slot_mapping.numel() <= 1 || slot_mapping.stride(0) == 1,
              "slot_mapping must be contiguous");
  if (rows.size(0) == 0) return;
  c10::hip::HIPGuard guard(dev.index());
  check(qsa_store_cache_rows(cache.data_ptr(), sdim(cache, 0), sdim(cache, 1),
                             (int)cache.size(0), (int)cache.size(1), (int)cache.size(3),
                             at_elem<int64_t>(slot_mapping), rows.data_ptr(), sdim(rows, 0),
                             (int)rows.size(0), stream_of(dev)),
        "qsa_store_cache_rows");
}

void compress_groups_impl(const Tensor& raw_keys, const OptTensor& raw_positions,
                          const Tensor& state_cache, const OptTensor& rope_cache,
                          const Tensor& state_table, const Tensor& token_to_req,
                          const Tensor& query_start_loc, const Tensor& logical_positions,
                          const Tensor& compressed_slots, int64_t ratio, const Tensor& pooled,
                          const Tensor& first_positions) {
  const auto dev = on_gpu({&raw_keys, opt(raw_positions), &state_cache, opt(rope_cache),
                           &state_table, &token_to_req, &query_start_loc, &logical_positions,
                           &compressed_slots, &pooled, &first_positions});
  dtype(raw_keys, at::kBFloat16, "raw_keys");
  QSA_REQUIRE(raw_keys.dim() == 3 && raw_keys.size(1) == 1 && raw_keys.stride(2) == 1,
              "raw_keys must be [rows, 1, dim] with unit dim stride");
  const int64_t dim = raw_keys.size(2);
  dtype(state_cache, at::kBFloat16, "compressor_state_cache");
  QSA_REQUIRE(state_cache.dim() == 4 && state_cache.size(2) == 1 && state_cache.stride(3) == 1 &&
                  state_cache.size(3) >= dim,
              "compressor_state_cache must be [blocks, ring, 1, >= dim] with unit dim stride");
  vec(token_to_req, at::kInt, "token_to_req");
  const int64_t rows = token_to_req.numel();
  vec(query_start_loc, at::kInt, "query_start_loc");
  dtype(state_table, at::kInt, "compressor_state_block_table");
  QSA_REQUIRE(state_table.dim() == 2 && state_table.size(0) >= query_start_loc.numel() - 1,
              "compressor_state_block_table must be [requests, width]");
  for (auto [t, name] : {std::pair<const Tensor*, const char*>{&logical_positions,
                                                               "logical_positions"},
                         {&compressed_slots, "compressed_slots"}}) {
    positions(*t, rows, name);
    QSA_REQUIRE(t->numel() <= 1 || t->stride(0) == 1, name, " must be contiguous");
  }
  QSA_REQUIRE(raw_keys.size(0) >= rows, "raw_keys has fewer rows than token_to_req");
  dtype(pooled, at::kBFloat16, "pooled");
  QSA_REQUIRE(pooled.dim() == 3 && pooled.size(0) >= rows && pooled.size(2) == dim &&
                  pooled.stride(2) == 1,
              "pooled must be [rows, 1, dim]");
  dtype(first_positions, at::kLong, "first_positions");
  QSA_REQUIRE(first_positions.dim() == 2 && first_positions.size(1) >= 3,
              "first_positions must be [rows, 3]");
  int64_t rp0 = 0, rp2 = 0;
  if (rope_cache) {
    dtype(*rope_cache, at::kLong, "rope_cache");
    QSA_REQUIRE(rope_cache->dim() == 4 && rope_cache->size(3) >= 3,
                "rope_cache must be [blocks, ring, 1, >= 3] int64");
    QSA_REQUIRE(raw_positions.has_value(), "raw_positions are needed with rope_cache");
    dtype(*raw_positions, at::kLong, "raw_positions");
    QSA_REQUIRE(raw_positions->dim() == 3 && raw_positions->size(2) >= 3,
                "raw_positions must be [rows, 1, >= 3] int64");
    rp0 = sdim(*raw_positions, 0);
    rp2 = sdim(*raw_positions, 2);
  }
  if (rows == 0) return;
  c10::hip::HIPGuard guard(dev.index());
  const Tensor* rc = opt(rope_cache);
  check(qsa_compress_groups(
            raw_keys.data_ptr(), sdim(raw_keys, 0),
            rc ? at_elem<int64_t>(*raw_positions) : nullptr, rp0, rp2, state_cache.data_ptr(),
            sdim(state_cache, 0), sdim(state_cache, 1), (int)state_cache.size(1),
            (int)state_cache.size(0), rc ? at_elem<int64_t>(*rc) : nullptr,
            rc ? sdim(*rc, 0) : 0, rc ? sdim(*rc, 1) : 0, rc ? sdim(*rc, 3) : 0,
            at_elem<int32_t>(state_table), sdim(state_table, 0), at_elem<int32_t>(token_to_req),
            at_elem<int32_t>(query_start_loc), (int)query_start_loc.numel() - 1,
            at_elem<int64_t>(logical_positions), at_elem<int64_t>(compressed_slots), (int)rows,
            (int)dim, (int)ratio, pooled.data_ptr(), sdim(pooled, 0),
            at_elem<int64_t>(first_positions), sdim(first_positions, 0),
            first_positions.stride(1), stream_of(dev)),
        "qsa_compress_groups");
}

void expand_block_indices_impl(const Tensor& block_indices, const Tensor& pos,
                               const Tensor& sequence_lengths, const Tensor& token_to_req,
                               const Tensor& table, const Tensor& output, const Tensor& counts,
                               int64_t ratio, int64_t topk, int64_t page_size, bool physical,
                               bool store_counts) {
  const auto dev = on_gpu({&block_indices, &pos, &sequence_lengths, &token_to_req, &table,
                           &output, &counts});
  dtype(block_indices, at::kInt, "block_indices");
  QSA_REQUIRE(block_indices.dim() == 2, "block_indices must be [rows, blocks]");
  const int64_t rows = block_indices.size(0);
  positions(pos, rows, "query_positions");
  vec(sequence_lengths, at::kInt, "sequence_lengths");
  vec(token_to_req, at::kInt, "token_to_req", rows);
  dtype(output, at::kInt, "output");
  QSA_REQUIRE(output.dim() == 2 && output.size(0) >= rows, "output must be [rows, width]");
  if (physical) table2d(table, "main_block_table");
  if (store_counts) vec(counts, at::kInt, "valid_counts_out", rows);
  if (rows == 0) return;
  c10::hip::HIPGuard guard(dev.index());
  check(qsa_expand_block_indices(
            at_elem<int32_t>(block_indices), sdim(block_indices, 0), sdim(block_indices, 1),
            (int)block_indices.size(1), (int)rows, (int)topk, at_elem<int64_t>(pos),
            at_elem<int32_t>(sequence_lengths), (int)sequence_lengths.numel(),
            at_elem<int32_t>(token_to_req), physical ? at_elem<int32_t>(table) : nullptr,
            physical ? table.stride(0) : 0, physical ? (int)table.size(1) : 0,
            at_elem<int32_t>(output), sdim(output, 0), output.stride(1), (int)output.size(1),
            store_counts ? at_elem<int32_t>(counts) : nullptr, (int)ratio, (int)page_size,
            physical ? 1 : 0, store_counts ? 1 : 0, stream_of(dev)),
        "qsa_expand_block_indices");
}

}  // namespace

TORCH_LIBRARY_FRAGMENT(yulan_qsa_kernels, m) {
  // Reference schemas (ops/csrc/topk.cu:549-552).
  m.def("topk(Tensor scores, Tensor lengths, Tensor(a!) output) -> ()");
  m.def(
      "topk_expand(Tensor scores, Tensor lengths, Tensor positions, Tensor sequence_lengths, "
      "Tensor token_to_req, Tensor table, Tensor(a!) output, Tensor(b!) counts, int ratio, "
      "int page_size, bool physical, bool store_counts) -> ()");
  // This library's own ops.
  m.def(
      "indexer_prepare(Tensor index_qk, Tensor positions, Tensor q_norm_weight, "
      "Tensor k_norm_weight, Tensor cos_sin, float eps, Tensor(a!) index_q_out, "
      "Tensor(b!) state_cache, Tensor state_slots, Tensor state_table, Tensor query_start_loc, "
      "Tensor logical_positions, Tensor(c!) compressed_cache, Tensor compressed_slots, "
      "Tensor k_work, Tensor main_key, Tensor main_value, Tensor(d!) main_key_cache, "
      "Tensor(e!) main_value_cache, Tensor main_slots, int num_index_heads, "
      "int index_head_dim, int rotary_dim, int compress_ratio) -> ()");
  m.def("store_cache_rows(Tensor(a!) cache, Tensor slot_mapping, Tensor rows) -> ()");
  m.def(
      "compress_groups(Tensor raw_keys, Tensor? raw_positions, Tensor state_cache, "
      "Tensor? rope_cache, Tensor state_table, Tensor token_to_req, Tensor query_start_loc, "
      "Tensor logical_positions, Tensor compressed_slots, int ratio, Tensor(a!) pooled, "
      "Tensor(b!) first_positions) -> ()");
  m.def(
      "expand_block_indices(Tensor block_indices, Tensor positions, Tensor sequence_lengths, "
      "Tensor token_to_req, Tensor table, Tensor(a!) output, Tensor(b!) counts, int ratio, "
      "int topk, int page_size, bool physical, bool store_counts) -> ()");
  m.def(
      "indexer_norm_rope(Tensor values, Tensor weight, Tensor positions, Tensor cos_sin, "
      "float eps, int rotary_dim, Tensor(a!) out) -> ()");
  m.def(
      "indexer_decode(Tensor q, Tensor k_cache, Tensor page_table, Tensor visible, "
      "Tensor(a!) logits, int decode_query_len) -> ()");
  m.def(
      "indexer_prefill(Tensor q, Tensor k_cache, Tensor page_table, Tensor query_start_loc, "
      "Tensor visible, Tensor(a!) logits, int query_offset, int num_rows, "
      "int max_query_len) -> ()");
  m.def(
      "select_decode(Tensor q, Tensor k_cache, Tensor page_table, Tensor visible, "
      "Tensor positions, Tensor sequence_lengths, Tensor token_to_req, Tensor(a!) output, "
      "Tensor? table, Tensor(b!)? counts, int ratio, int decode_query_len, int columns, "
      "int page_size, int cap_bytes) -> ()");
  m.def(
      "select_prefill(Tensor q, Tensor k_cache, Tensor page_table, Tensor query_start_loc, "
      "Tensor visible, Tensor positions, Tensor sequence_lengths, Tensor token_to_req, "
      "Tensor(a!) output, Tensor? table, Tensor(b!)? counts, int ratio, int max_query_len, "
      "int width, int page_size, int cap_bytes) -> ()");
  m.def(
      "sparse_attention(Tensor q, Tensor k_cache, Tensor v_cache, Tensor indices, "
      "Tensor block_table, Tensor token_to_req, Tensor(a!) out, Tensor? output_gate, "
      "Tensor? valid_counts, bool indices_are_physical, int num_splits) -> ()");
  m.def(
      "sparse_attention_merge(Tensor partial_out, Tensor partial_lse, Tensor(a!) out, "
      "Tensor? output_gate) -> ()");
  m.def(
      "decode_select_attend(Tensor scores, Tensor lengths, Tensor positions, "
      "Tensor sequence_lengths, Tensor token_to_req, Tensor table, Tensor(a!) indices, "
      "Tensor(b!) counts, int ratio, Tensor q, Tensor k_cache, Tensor v_cache, Tensor(c!) out, "
      "Tensor? output_gate, int num_splits) -> ()");
}

TORCH_LIBRARY_IMPL(yulan_qsa_kernels, CUDA, m) {
  m.impl("topk", &topk_impl);
  m.impl("topk_expand", &topk_expand_impl);
  m.impl("indexer_prepare", &indexer_prepare_impl);
  m.impl("store_cache_rows", &store_cache_rows_impl);
  m.impl("compress_groups", &compress_groups_impl);
  m.impl("expand_block_indices", &expand_block_indices_impl);
  m.impl("indexer_norm_rope", &indexer_norm_rope_impl);
  m.impl("indexer_decode", &indexer_decode_impl);
  m.impl("indexer_prefill", &indexer_prefill_impl);
  m.impl("select_decode", &select_decode_impl);
  m.impl("select_prefill", &select_prefill_impl);
  m.impl("sparse_attention", &sparse_attention_impl);
  m.impl("sparse_attention_merge", &sparse_attention_merge_impl);
  m.impl("decode_select_attend", &decode_select_attend_impl);
}

// Shape-only tracing (fake / meta tensors): the ops mutate their outputs in
// place and return nothing, so there is nothing to compute.
TORCH_LIBRARY_IMPL(yulan_qsa_kernels, Meta, m) {
  m.impl("topk", [](const Tensor&, const Tensor&, const Tensor&) {});
  m.impl("topk_expand", [](const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                           const Tensor&, const Tensor&, const Tensor&, const Tensor&, int64_t,
                           int64_t, bool, bool) {});
  m.impl("indexer_decode",
         [](const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&, int64_t) {});
  m.impl("indexer_prefill", [](const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                               const Tensor&, const Tensor&, int64_t, int64_t, int64_t) {});
  m.impl("select_decode", [](const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                             const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                             const OptTensor&, const OptTensor&, int64_t, int64_t, int64_t,
                             int64_t, int64_t) {});
  m.impl("select_prefill", [](const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                              const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                              const Tensor&, const OptTensor&, const OptTensor&, int64_t, int64_t,
                              int64_t, int64_t, int64_t) {});
  m.impl("sparse_attention", [](const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                const Tensor&, const Tensor&, const Tensor&, const OptTensor&,
                                const OptTensor&, bool, int64_t) {});
  m.impl("sparse_attention_merge",
         [](const Tensor&, const Tensor&, const Tensor&, const OptTensor&) {});
  m.impl("decode_select_attend",
         [](const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&,
            const Tensor&, const Tensor&, const Tensor&, int64_t, const Tensor&, const Tensor&,
            const Tensor&, const Tensor&, const OptTensor&, int64_t) {});
  m.impl("indexer_prepare",
         [](const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&, double,
            const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&,
            const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&,
            const Tensor&, const Tensor&, const Tensor&, const Tensor&, int64_t, int64_t, int64_t,
            int64_t) {});
  m.impl("store_cache_rows", [](const Tensor&, const Tensor&, const Tensor&) {});
  m.impl("compress_groups", [](const Tensor&, const OptTensor&, const Tensor&, const OptTensor&,
                               const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                               const Tensor&, int64_t, const Tensor&, const Tensor&) {});
  m.impl("expand_block_indices",
         [](const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&,
            const Tensor&, const Tensor&, int64_t, int64_t, int64_t, bool, bool) {});
  m.impl("indexer_norm_rope", [](const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                 double, int64_t, const Tensor&) {});
}
