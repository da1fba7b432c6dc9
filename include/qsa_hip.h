/*
 * qsa_hip.h - C ABI of the MI355X (gfx950) QSA sparse-attention path.
 *
 * Plain pointers, sizes and element strides only; every entry point enqueues
 * its kernels on `stream` (a hipStream_t passed as void*) and never
 * synchronises or reads device data on the host. Entry points return QSA_OK or
 * a negative status; qsa_last_error() gives the message of the calling thread's
 * last failure.
 *
 * Each entry point replaces one interface of the reference vLLM plugin
 * (clotholza/qsa_vllm, package yulan_qsa_vllm); the citation names the file
 * and lines whose behaviour it reproduces.
 */
#ifndef QSA_HIP_H
#define QSA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QSA_OK 0
#define QSA_ERR_INVALID (-1)     /* bad shape, stride, pointer or size */
#define QSA_ERR_UNSUPPORTED (-2) /* valid input this library has no kernel for */
#define QSA_ERR_HIP (-3)         /* a HIP runtime call failed */
#define QSA_ERR_WORKSPACE (-4)   /* workspace missing or too small */

/* Message of the calling thread's last failed call ("" if none). */
const char* qsa_last_error(void);

/* ABI version of this library (increments on any signature change). */
int qsa_abi_version(void);

/* ------------------------------------------------------------------------ */
/* Kernel 2: exact top-k block selection                                     */
/* ------------------------------------------------------------------------ */

/* Bytes of device workspace qsa_topk / qsa_topk_expand need for this shape
 * (0 when the row fits the single-pass kernel). */
size_t qsa_topk_workspace_bytes(int rows, int cols, int topk);

/*
 * Replaces torch.ops.yulan_qsa_kernels.topk (ops/csrc/topk.cu:527-545,
 * schema :549, Python wrapper ops/topk.py:25-26).
 *
 * scores [rows, cols] fp32 (row stride score_row_stride, unit column stride),
 * lengths [rows] int32, output [rows, topk] int32 (unit column stride).
 * Per row, L = lengths[r]: L <= topk writes ids 0..L-1 then -1; otherwise the
 * topk ids whose scores have the largest raw fp32 bit patterns read as uint32
 * (lowest id first among equal patterns), in ascending id order.
 */
int qsa_topk(const float* scores, int64_t score_row_stride, int rows, int cols,
             const int32_t* lengths, int32_t* output, int64_t output_row_stride, int topk,
             void* workspace, size_t workspace_bytes, void* stream);

/*
 * Replaces torch.ops.yulan_qsa_kernels.topk_expand (ops/csrc/topk.cu:470-525,
 * schema :550-552, Python wrapper ops/topk.py:29-39).
 *
 * Selection as qsa_topk with topk = output_width / ratio, then each selected
 * block b at rank i expands to tokens b*ratio + o at output columns
 * i*ratio + o, followed by the visible incomplete causal tail, then -1.
 * physical != 0 maps tokens through `table` [num_requests, table_width] to
 * slots page*page_size + offset; store_counts != 0 writes counts[rows].
 * positions are int64; all other index arrays int32 and contiguous.
 */
int qsa_topk_expand(const float* scores, int64_t score_row_stride, int rows, int cols,
                    const int32_t* lengths, const int64_t* positions,
                    const int32_t* sequence_lengths, int num_requests,
                    const int32_t* token_to_req,
                    const int32_t* table, int64_t table_row_stride, int table_width,
                    int32_t* output, int64_t output_row_stride, int64_t output_col_stride,
                    int output_width, int32_t* counts, int ratio, int page_size,
                    int physical, int store_counts,
                    void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Kernel 0: indexer preparation and cache producers                          */
/* ------------------------------------------------------------------------ */

/*
 * Replaces the launch of _qsa_prepare_kernel in qsa_prepare
 * (ops/prepare.py:177-225; kernel :49-174, numerics :16-46).
 *
 * index_qk [num_tokens, (num_index_heads + 1) * index_head_dim] bf16 (token
 * stride index_token_stride, unit dim stride): the index queries, then the
 * raw index key. positions / logical_positions int64; slot mappings int64
 * (-1: no write); state_table, query_start_loc, k_work int32; k_work is
 * [num_k_work, 2] (request, group within request), request < 0 for padding.
 * Writes index_q_out [num_tokens, num_index_heads, index_head_dim] (RMSNorm +
 * partial RoPE of every query head), one normalised mean-pooled key per
 * compression group into compressed_cache [blocks, comp_page_size, dim],
 * the last min(query_len, state_size) raw keys of each request into its ring
 * state_cache [blocks, state_size, dim], and main_key / main_value rows
 * [tokens, main_kv_heads, main_head_dim] into main_key_cache /
 * main_value_cache [blocks, main_page_size, main_kv_heads, main_head_dim].
 * cos_sin is [max_positions, rotary_dim] bf16 (cos, then sin). Strides are in
 * elements; every tensor is 16-byte aligned with unit dim stride.
 * index_head_dim and main_head_dim are 64 or 128; rotary_dim a multiple of 16.
 */
int qsa_indexer_prepare(const void* index_qk, int64_t index_token_stride, int num_tokens,
                        const int64_t* positions, int64_t position_stride,
                        const void* q_norm_weight, const void* k_norm_weight,
                        const void* cos_sin, int max_positions, float eps,
                        void* index_q_out,
                        void* state_cache, int64_t state_block_stride,
                        int64_t state_token_stride, int state_size, int num_state_blocks,
                        const int64_t* state_slots, const int32_t* state_table,
                        int64_t state_table_stride, const int32_t* query_start_loc,
                        const int64_t* logical_positions, int num_requests,
                        void* compressed_cache, int64_t comp_block_stride,
                        int64_t comp_token_stride, int comp_page_size, int num_comp_blocks,
                        const int64_t* compressed_slots, const int32_t* k_work, int num_k_work,
                        const void* main_key, int64_t main_key_token_stride,
                        int64_t main_key_head_stride,
                        const void* main_value, int64_t main_value_token_stride,
                        int64_t main_value_head_stride,
                        void* main_key_cache, int64_t main_key_cache_block_stride,
                        int64_t main_key_cache_token_stride, int64_t main_key_cache_head_stride,
                        void* main_value_cache, int64_t main_value_cache_block_stride,
                        int64_t main_value_cache_token_stride,
                        int64_t main_value_cache_head_stride,
                        const int64_t* main_slots, int main_page_size, int num_main_blocks,
                        int num_index_heads, int index_head_dim, int rotary_dim,
                        int compress_ratio, int main_kv_heads, int main_head_dim,
                        void* stream);

/*
 * Replaces indexer_norm_rope and its kernel _norm_rope
 * (ops/normalization.py:33-83): RMSNorm + partial RoPE of every row of
 * values [tokens, heads, dim] (unit dim stride) into a contiguous out.
 */
int qsa_indexer_norm_rope(const void* values, int64_t token_stride, int64_t head_stride,
                          int tokens, int heads, int dim, const void* weight,
                          const int64_t* positions, int64_t position_stride,
                          const void* cos_sin, int max_positions, float eps, int rotary_dim,
                          void* out, void* stream);

/*
 * Replaces qsa_store_cache_rows and its kernel _store_qsa_rows_kernel
 * (ops/qsa.py:366-401, 691-706): rows [num_rows, width] bf16 into
 * cache[slot / page_size, slot % page_size, 0, :width] for
 * 0 <= slot_mapping[r] < num_blocks * page_size (int64 slots).
 */
int qsa_store_cache_rows(void* cache, int64_t cache_block_stride, int64_t cache_token_stride,
                         int num_blocks, int page_size, int width,
                         const int64_t* slot_mapping, const void* rows, int64_t row_stride,
                         int num_rows, void* stream);

/*
 * Replaces qsa_compress_groups_with_ratio and its kernel
 * _compress_qsa_groups_kernel (ops/qsa.py:403-549, 709-750): for each row
 * (token) that closes a group with a compressed slot, the bf16 mean of the
 * compress_ratio raw keys ending at its position (this step's rows, or the
 * request's ring before the chunk; fp32 sum in member order), else 0; and the
 * group's first position in 3 int64 columns, read from raw_positions /
 * rope_positions when rope_positions is given. Every row of pooled and
 * first_positions is written.
 */
int qsa_compress_groups(const void* raw_keys, int64_t raw_row_stride,
                        const int64_t* raw_positions, int64_t raw_pos_row_stride,
                        int64_t raw_pos_dim_stride, const void* state_cache,
                        int64_t state_block_stride, int64_t state_token_stride, int state_size,
                        int num_state_blocks, const int64_t* rope_positions,
                        int64_t rope_block_stride, int64_t rope_token_stride,
                        int64_t rope_dim_stride, const int32_t* state_table,
                        int64_t state_table_stride, const int32_t* token_to_req,
                        const int32_t* query_start_loc, int num_requests,
                        const int64_t* logical_positions, const int64_t* compressed_slots,
                        int rows, int head_dim, int compress_ratio, void* pooled,
                        int64_t pooled_row_stride, int64_t* first_positions,
                        int64_t first_positions_row_stride, int64_t first_positions_col_stride,
                        void* stream);

/* ------------------------------------------------------------------------ */
/* Kernel 1: indexer scoring                                                 */
/* ------------------------------------------------------------------------ */

/*
 * Replaces the decode scoring launch of qsa_select_paged_decode
 * (ops/indexer.py:24-114, launch :259-272).
 *
 * q [rows, num_heads, head_dim] bf16 (unit dim stride); k_cache
 * [num_blocks, cache_page, (1,) head_dim] bf16 (unit dim stride);
 * page_table [rows / decode_query_len, table_width] int32; visible [rows].
 * Writes logits[r, c] = head_dim^-0.5 * sum_h relu(q[r,h,:] . K[c,:]) for
 * c < min(visible[r], table_width * cache_page, logits_cols); other columns
 * are left untouched.
 */
int qsa_indexer_decode(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                       int rows, int num_heads, int head_dim,
                       const void* k_cache, int64_t cache_block_stride,
                       int64_t cache_token_stride, int num_blocks, int cache_page,
                       const int32_t* page_table, int64_t table_row_stride, int table_width,
                       const int32_t* visible, int decode_query_len,
                       float* logits, int64_t logits_row_stride, int logits_cols,
                       void* stream);

/*
 * Rows per logits span of the prefill selection (ops/indexer.py:324-329
 * chunks rows by QSA_INDEXER_WORKSPACE_MB): the largest count within
 * cap_bytes of fp32 logits of logits_cols columns, rounded down to whole
 * launch rounds (one 32-row workgroup per compute unit) when the cap allows
 * one. Only the launch count differs from the reference's chunking; every
 * row's selection is the same.
 */
int qsa_indexer_prefill_span_rows(int logits_cols, int64_t cap_bytes);

/*
 * Replaces _prefill_logits (ops/indexer.py:117-223, launch :282-302).
 *
 * q / visible are indexed by the prefill-relative absolute row; logits rows by
 * row - query_offset for the num_rows rows of this chunk. Request req covers
 * rows [query_start_loc[req] - query_start_loc[0],
 * query_start_loc[req+1] - query_start_loc[0]) and uses page_table[req].
 */
int qsa_indexer_prefill(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                        int num_heads, int head_dim,
                        const void* k_cache, int64_t cache_block_stride,
                        int64_t cache_token_stride, int num_blocks, int cache_page,
                        const int32_t* page_table, int64_t table_row_stride, int table_width,
                        int num_requests, const int32_t* query_start_loc,
                        const int32_t* visible, int query_offset, int num_rows,
                        int max_query_len,
                        float* logits, int64_t logits_row_stride, int logits_cols,
                        void* stream);

/*
 * Replaces expand_qsa_block_indices_cuda and its kernel
 * _expand_qsa_indices_kernel (ops/qsa.py:18-106, 552-591): the expansion of
 * qsa_topk_expand applied to caller-chosen block ids (block_indices
 * [rows, >= topk] int32, rank i = column i, -1 for none) instead of a top-k.
 */
int qsa_expand_block_indices(const int32_t* block_indices, int64_t block_row_stride,
                             int64_t block_col_stride, int block_cols, int rows, int topk,
                             const int64_t* positions, const int32_t* sequence_lengths,
                             int num_requests, const int32_t* token_to_req,
                             const int32_t* table, int64_t table_row_stride, int table_width,
                             int32_t* output, int64_t output_row_stride,
                             int64_t output_col_stride, int output_width, int32_t* counts,
                             int ratio, int page_size, int physical, int store_counts,
                             void* stream);

/* ------------------------------------------------------------------------ */
/* Kernel 3: bf16 paged sparse GQA attention                                 */
/* ------------------------------------------------------------------------ */

/* Split count the library picks for this shape (use_decode_kernel as in
 * ops/qsa.py:620-645: decode rows iterate only their valid count). */
int qsa_sparse_attention_splits(int rows, int num_q_heads, int num_kv_heads, int head_dim,
                                int width, int use_decode_kernel);

/* Bytes of fp32 split partials (output + log2-LSE) for num_splits > 1. */
size_t qsa_sparse_attention_workspace_bytes(int rows, int num_q_heads, int head_dim,
                                            int num_splits);

/*
 * Replaces qsa_sparse_paged_attention (ops/qsa.py:594-688) and its kernels
 * _qsa_sparse_paged_gqa_splitk_kernel (:109-303) and _qsa_merge_splitk_kernel
 * (:306-362).
 *
 * q [rows, Hq, D] bf16; k_cache / v_cache [num_blocks, page_size, Hkv, D] bf16
 * views with arbitrary block/token/head strides and unit dim stride;
 * indices [rows, width] int32 (unit column stride): physical slots
 * (page*page_size + offset) when indices_are_physical, else logical token ids
 * mapped through block_table[token_to_req[r]]. valid_counts (may be NULL)
 * limits row r to its first valid_counts[r] entries. Head h attends with kv
 * head h / (Hq / Hkv). out [rows, Hq, D] bf16 (unit dim stride); gate (may be
 * NULL) multiplies bf16(out) by sigmoid(gate). num_splits > 1 needs a workspace
 * of qsa_sparse_attention_workspace_bytes(). Strides are in elements.
 */
int qsa_sparse_attention(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                         int rows, int num_q_heads, int head_dim,
                         const void* k_cache, int64_t k_block_stride, int64_t k_token_stride,
                         int64_t k_head_stride,
                         const void* v_cache, int64_t v_block_stride, int64_t v_token_stride,
                         int64_t v_head_stride,
                         int num_blocks, int page_size, int num_kv_heads,
                         const int32_t* indices, int64_t indices_row_stride, int width,
                         const int32_t* block_table, int64_t table_row_stride,
                         int table_width, int num_requests,
                         const int32_t* token_to_req, const int32_t* valid_counts,
                         void* out, int64_t out_row_stride, int64_t out_head_stride,
                         const void* gate, int64_t gate_row_stride, int64_t gate_head_stride,
                         int64_t gate_dim_stride,
                         int indices_are_physical, int num_splits,
                         void* workspace, size_t workspace_bytes, void* stream);

/* Whether qsa_decode_select_attention runs this decode batch shape as one
 * launch (plus the split merge) over token-major K/V views spanning under
 * 4 GB per kv head; 0: it runs the top-k and the attention as two calls. */
int qsa_decode_select_attention_fuses(int rows, int cols, int width, int ratio,
                                      int num_q_heads, int num_kv_heads, int head_dim);

/* Bytes of workspace qsa_decode_select_attention needs: the larger of the
 * top-k's (qsa_topk_workspace_bytes of topk = width / ratio) and the split
 * partials' (qsa_sparse_attention_workspace_bytes). */
size_t qsa_decode_select_attention_workspace_bytes(int rows, int cols, int width, int ratio,
                                                   int num_q_heads, int head_dim,
                                                   int num_splits);

/*
 * The decode half of a QSA layer after scoring: replaces the top-k +
 * expansion that qsa_select_paged_decode runs on the logits
 * (ops/indexer.py:241-279, attention.py:128-145) followed by the backend's
 * sparse attention over the selection (backend.py:49-68 with
 * indices_are_physical and valid_counts), for a batch of decode rows.
 *
 * Results equal qsa_topk_expand(scores, ..., output = indices,
 * output_col_stride = 1, output_width = width, counts, ratio, page_size,
 * physical = 1, store_counts = 1) followed by qsa_sparse_attention(q, ...,
 * indices, width, block_table, ..., valid_counts = counts,
 * indices_are_physical = 1, num_splits): the selection (indices, counts) and
 * the attention output. Batches of fewer than 1024 rows of at most 2048
 * logits columns whose attention runs 8-wave workgroups over buffer-addressed
 * caches with at most 2 kv heads per workgroup run both in one launch (plus
 * the split merge), each workgroup selecting its row into LDS; other shapes
 * run the two calls. num_splits <= 0 takes qsa_sparse_attention_splits'
 * choice. The workspace is qsa_decode_select_attention_workspace_bytes().
 */
int qsa_decode_select_attention(const float* scores, int64_t score_row_stride, int rows,
                                int cols, const int32_t* lengths, const int64_t* positions,
                                const int32_t* sequence_lengths, int num_requests,
                                const int32_t* token_to_req, const int32_t* block_table,
                                int64_t table_row_stride, int table_width, int ratio,
                                int32_t* indices, int64_t indices_row_stride, int width,
                                int32_t* counts,
                                const void* q, int64_t q_row_stride, int64_t q_head_stride,
                                int num_q_heads, int head_dim,
                                const void* k_cache, int64_t k_block_stride,
                                int64_t k_token_stride, int64_t k_head_stride,
                                const void* v_cache, int64_t v_block_stride,
                                int64_t v_token_stride, int64_t v_head_stride,
                                int num_blocks, int page_size, int num_kv_heads,
                                void* out, int64_t out_row_stride, int64_t out_head_stride,
                                const void* gate, int64_t gate_row_stride,
                                int64_t gate_head_stride, int64_t gate_dim_stride,
                                int num_splits, void* workspace, size_t workspace_bytes,
                                void* stream);

/* Bytes of device scratch qsa_sparse_attention_noalloc holds per GPU. */
#define QSA_SPARSE_ATTENTION_SCRATCH_BYTES ((size_t)32 << 20)

/*
 * No counterpart in the reference: qsa_sparse_attention for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Same arguments and results, minus
 * the workspace: the split partials live in a device array of
 * QSA_SPARSE_ATTENTION_SCRATCH_BYTES (32 MiB) that the library holds on each
 * GPU it runs on until the process ends. Calls whose partials
 * (qsa_sparse_attention_workspace_bytes) exceed it fail with
 * QSA_ERR_WORKSPACE. The call allocates nothing. Every call on one GPU shares
 * that GPU's array, so calls that overlap in time on one GPU (different
 * streams without ordering between them) race. `stream` must belong to the
 * current device.
 */
int qsa_sparse_attention_noalloc(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                                 int rows, int num_q_heads, int head_dim,
                                 const void* k_cache, int64_t k_block_stride,
                                 int64_t k_token_stride, int64_t k_head_stride,
                                 const void* v_cache, int64_t v_block_stride,
                                 int64_t v_token_stride, int64_t v_head_stride,
                                 int num_blocks, int page_size, int num_kv_heads,
                                 const int32_t* indices, int64_t indices_row_stride, int width,
                                 const int32_t* block_table, int64_t table_row_stride,
                                 int table_width, int num_requests,
                                 const int32_t* token_to_req, const int32_t* valid_counts,
                                 void* out, int64_t out_row_stride, int64_t out_head_stride,
                                 const void* gate, int64_t gate_row_stride,
                                 int64_t gate_head_stride, int64_t gate_dim_stride,
                                 int indices_are_physical, int num_splits, void* stream);

/*
 * Replaces _qsa_merge_splitk_kernel (ops/qsa.py:306-362) as a standalone call:
 * partial_out [num_splits, rows, Hq, D] fp32, partial_lse [num_splits, rows, Hq]
 * fp32 (log2 domain, -inf for empty splits) -> out bf16 (+ optional gate).
 */
int qsa_sparse_attention_merge(const float* partial_out, const float* partial_lse,
                               int num_splits, int rows, int num_q_heads, int head_dim,
                               void* out, int64_t out_row_stride, int64_t out_head_stride,
                               const void* gate, int64_t gate_row_stride,
                               int64_t gate_head_stride, int64_t gate_dim_stride,
                               void* stream);

/* ------------------------------------------------------------------------ */
/* Hybrid decoder layers around the path (the model's other token mixers)    */
/* ------------------------------------------------------------------------ */

/*
 * Replaces YuLanGatedNorm.forward (model.py:85-98) with vLLM's fused
 * residual-add RMSNorm inside: when residual_in is given, residual_out =
 * bf16(x + residual_in) (may alias residual_in) and the norm runs on it;
 * out = n * bf16(sigmoid(gate_up(silu(gate_down(n))) + bias)) with
 * n = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * weight). gate_down [rank, hidden],
 * gate_up [hidden, rank], rank 16, hidden a multiple of 512 up to 4096.
 */
int qsa_gated_norm(const void* x, int64_t x_stride, const void* residual_in,
                   int64_t residual_in_stride, void* residual_out, int64_t residual_out_stride,
                   const void* weight, const void* gate_down, const void* gate_up,
                   const void* gate_up_bias, void* out, int64_t out_stride, int rows,
                   int hidden, int rank, float eps, void* workspace, size_t workspace_bytes,
                   void* stream);

/* Workspace qsa_gated_norm needs for `rows` tokens: 0 for every shape (small
 * batches, under 1024 tokens, run one workgroup per token; larger ones
 * 16-token tiles). Kept so callers that size a workspace keep working. */
size_t qsa_gated_norm_workspace_bytes(int rows, int hidden);

/*
 * Replaces the SiluAndMul activation of Qwen2MoeMLP (model.py:211-217, vLLM):
 * out[t, i] = bf16(silu(gu[t, i]) * gu[t, intermediate + i]) in fp32.
 */
int qsa_silu_mul(const void* gate_up, int64_t gate_up_stride, void* out, int64_t out_stride,
                 int rows, int intermediate, void* stream);

/*
 * The GDN token mixer of the linear-attention layers (model.py:205-212:
 * vLLM's QwenGatedDeltaNetAttention). Sequences are consecutive token ranges
 * [query_start_loc[s], query_start_loc[s+1]) with state slot slots[s]
 * (slots outside [0, num_slots) have no state: zero initial state, nothing
 * stored). Projection rows are grouped per key head [q, k, v (r heads),
 * z (r heads)] (qkvz) and [b (r), a (r)] (ba); head dims 128.
 *
 * qsa_gdn_prep: causal depthwise conv (width conv_kernel, weights
 * [channels, K]) over each sequence's inputs, the conv state [slots, K-1,
 * channels] supplying the inputs before the chunk, SiLU, bf16; q_out/k_out
 * [tokens, key_heads, 128] fp32 l2-normalised (q times 128^-1/2); v_out
 * [tokens, value_heads, 128] bf16; g_out = -exp(A_log) softplus(a + dt_bias),
 * beta_out = sigmoid(b), [tokens, value_heads] fp32.
 */
int qsa_gdn_prep(const void* qkvz, int64_t qkvz_stride, const void* ba, int64_t ba_stride,
                 const void* conv_weight, const void* conv_state, int num_slots,
                 const int32_t* query_start_loc, const int32_t* token_to_seq,
                 const int64_t* slots, int num_seqs, const float* A_log, const float* dt_bias,
                 int key_heads, int value_heads, int head_dim, int conv_kernel, int tokens,
                 float* q_out, float* k_out, void* v_out, float* g_out, float* beta_out,
                 void* stream);

/* The conv state after the step: each sequence's last K-1 inputs. Run after
 * qsa_gdn_prep of the same step (which reads the old state). Sequences whose
 * range leaves [0, tokens) are skipped (also by qsa_gdn_recurrence). */
int qsa_gdn_conv_state(const void* qkvz, int64_t qkvz_stride, int tokens, void* conv_state,
                       int num_slots, const int32_t* query_start_loc, const int64_t* slots,
                       int num_seqs, int key_heads, int value_heads, int head_dim,
                       int conv_kernel, void* stream);

/* Gated delta rule over each sequence's tokens in order, the state [slots,
 * value_heads, 128, 128] fp32 updated in place: S <- e^g S,
 * u = beta (v - S^T k), S <- S + k u^T, o = S^T q; o [tokens, value_heads, 128]
 * bf16. Value head h reads key head h / (value_heads / key_heads).
 * max_seq_tokens: the longest sequence's token count if the caller knows it,
 * else -1. Below 16 (a decode batch) the chunked kernel for sequences of 16+
 * tokens is not launched and the per-token kernel takes every sequence, so a
 * bound that is too small still gives a result within the same tolerance of
 * the per-token rule (not bit-identical: the per-token kernel is fp32
 * throughout, the chunked one multiplies in bf16), only slower. */
int qsa_gdn_recurrence(const float* q, const float* k, const void* v, const float* g,
                       const float* beta, int tokens, float* state, int num_slots,
                       const int32_t* query_start_loc, const int64_t* slots, int num_seqs,
                       int key_heads, int value_heads, int head_dim, int max_seq_tokens, void* o,
                       void* stream);

/* Gated RMSNorm of the GDN output: y = bf16(rmsnorm(o) * weight * silu(z)) per
 * (token, value head), z read from the qkvz projection rows. Tensors 16-byte
 * aligned, qkvz_stride a multiple of 8 elements. */
int qsa_gdn_gated_norm(const void* o, const void* qkvz, int64_t qkvz_stride, const void* weight,
                       float eps, int tokens, int key_heads, int value_heads, int head_dim,
                       void* y, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QSA_HIP_H */
