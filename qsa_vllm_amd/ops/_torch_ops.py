"""``torch.ops.yulan_qsa_kernels`` registrations backed by ``libqsa_hip.so``.

``topk`` and ``topk_expand`` keep the reference schemas verbatim
(ops/csrc/topk.cu:548-557 of the reference plugin). The indexer scoring,
sparse attention and split merge are new ops in the same namespace. Every
implementation validates dtypes/devices/layouts (raising RuntimeError like the
reference's ``TORCH_CHECK``/``data_ptr<T>()`` failures), then calls the C ABI
on the current stream of the tensor's device. Nothing here synchronises.
"""

from __future__ import annotations

import ctypes

import torch

from .. import _lib

_NS = "yulan_qsa_kernels"

_SCHEMAS = {
    # Reference schemas (ops/csrc/topk.cu:549-552).
    "topk": "topk(Tensor scores, Tensor lengths, Tensor(a!) output) -> ()",
    "topk_expand": (
        "topk_expand(Tensor scores, Tensor lengths, Tensor positions, Tensor sequence_lengths, "
        "Tensor token_to_req, Tensor table, Tensor(a!) output, Tensor(b!) counts, "
        "int ratio, int page_size, bool physical, bool store_counts) -> ()"),
    # New ops of this build.
    "indexer_prepare": (
        "indexer_prepare(Tensor index_qk, Tensor positions, Tensor q_norm_weight, "
        "Tensor k_norm_weight, Tensor cos_sin, float eps, Tensor(a!) index_q_out, "
        "Tensor(b!) state_cache, Tensor state_slots, Tensor state_table, Tensor query_start_loc, "
        "Tensor logical_positions, Tensor(c!) compressed_cache, Tensor compressed_slots, "
        "Tensor k_work, Tensor main_key, Tensor main_value, Tensor(d!) main_key_cache, "
        "Tensor(e!) main_value_cache, Tensor main_slots, int num_index_heads, "
        "int index_head_dim, int rotary_dim, int compress_ratio) -> ()"),
    "store_cache_rows": "store_cache_rows(Tensor(a!) cache, Tensor slot_mapping, Tensor rows) -> ()",
    "compress_groups": (
        "compress_groups(Tensor raw_keys, Tensor? raw_positions, Tensor state_cache, "
        "Tensor? rope_cache, Tensor state_table, Tensor token_to_req, Tensor query_start_loc, "
        "Tensor logical_positions, Tensor compressed_slots, int ratio, Tensor(a!) pooled, "
        "Tensor(b!) first_positions) -> ()"),
    "expand_block_indices": (
        "expand_block_indices(Tensor block_indices, Tensor positions, Tensor sequence_lengths, "
        "Tensor token_to_req, Tensor table, Tensor(a!) output, Tensor(b!) counts, int ratio, "
        "int topk, int page_size, bool physical, bool store_counts) -> ()"),
    "indexer_norm_rope": (
        "indexer_norm_rope(Tensor values, Tensor weight, Tensor positions, Tensor cos_sin, "
        "float eps, int rotary_dim, Tensor(a!) out) -> ()"),
    "indexer_decode": (
        "indexer_decode(Tensor q, Tensor k_cache, Tensor page_table, Tensor visible, "
        "Tensor(a!) logits, int decode_query_len) -> ()"),
    "indexer_prefill": (
        "indexer_prefill(Tensor q, Tensor k_cache, Tensor page_table, Tensor query_start_loc, "
        "Tensor visible, Tensor(a!) logits, int query_offset, int num_rows, "
        "int max_query_len) -> ()"),
    "sparse_attention": (
        "sparse_attention(Tensor q, Tensor k_cache, Tensor v_cache, Tensor indices, "
        "Tensor block_table, Tensor token_to_req, Tensor(a!) out, Tensor? output_gate, "
        "Tensor? valid_counts, bool indices_are_physical, int num_splits) -> ()"),
    "sparse_attention_merge": (
        "sparse_attention_merge(Tensor partial_out, Tensor partial_lse, Tensor(a!) out, "
        "Tensor? output_gate) -> ()"),
}


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _stride(t, d):
    """Stride of dim d, 0 for a size-1 dim (never used to address memory; views
    may carry any value there)."""
    return 0 if t.size(d) == 1 else t.stride(d)


def _require(cond, msg):
    if not cond:
        raise RuntimeError(f"{_NS}: {msg}")


def _on_gpu(*tensors):
    dev = None
    for t in tensors:
        if t is None:
            continue
        _require(t.is_cuda, f"expected a GPU tensor, got device {t.device}")
        if dev is None:
            dev = t.device
        _require(t.device == dev, "all tensors must be on the same device")
    return dev


def _dtype(t, dtype, name):
    _require(t.dtype == dtype, f"{name} must be {dtype}, got {t.dtype}")


def _vector(t, dtype, name, min_len=None):
    _dtype(t, dtype, name)
    _require(t.dim() == 1, f"{name} must be 1-D")
    _require(t.numel() <= 1 or t.stride(0) == 1, f"{name} must be contiguous")
    if min_len is not None:
        _require(t.numel() >= min_len, f"{name} has {t.numel()} entries, need {min_len}")


def _workspace(nbytes, device):
    if nbytes == 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


# --- topk / topk_expand -----------------------------------------------------

def _topk_impl(scores, lengths, output):
    dev = _on_gpu(scores, lengths, output)
    _dtype(scores, torch.float32, "scores")
    _require(scores.dim() == 2 and (scores.size(1) <= 1 or scores.stride(1) == 1),
             "scores must be [rows, cols] with unit column stride")
    _vector(lengths, torch.int32, "lengths", scores.size(0))
    _dtype(output, torch.int32, "output")
    _require(output.dim() == 2 and output.size(0) == scores.size(0)
             and (output.size(1) <= 1 or output.stride(1) == 1),
             "output must be [rows, topk] with unit column stride")
    rows, cols = scores.shape
    if rows == 0:
        return
    topk = output.size(1)
    lib = _lib.load()
    ws = _workspace(lib.qsa_topk_workspace_bytes(rows, cols, topk), dev)
    with torch.cuda.device(dev):
        _lib.call("qsa_topk", _ptr(scores), scores.stride(0), rows, cols, _ptr(lengths),
                  _ptr(output), output.stride(0), topk, _ptr(ws),
                  0 if ws is None else ws.numel(), _stream(dev))


def _topk_expand_impl(scores, lengths, positions, sequence_lengths, token_to_req, table,
                      output, counts, ratio, page_size, physical, store_counts):
    dev = _on_gpu(scores, lengths, positions, sequence_lengths, token_to_req, table, output, counts)
    _dtype(scores, torch.float32, "scores")
    _require(scores.dim() == 2 and (scores.size(1) <= 1 or scores.stride(1) == 1),
             "scores must be [rows, cols] with unit column stride")
    rows, cols = scores.shape
    _vector(lengths, torch.int32, "lengths", rows)
    _vector(positions, torch.int64, "positions", rows)
    _vector(sequence_lengths, torch.int32, "sequence_lengths")
    _vector(token_to_req, torch.int32, "token_to_req", rows)
    _dtype(output, torch.int32, "output")
    _require(output.dim() == 2 and output.size(0) == rows, "output must be [rows, width]")
    _require(ratio > 0, "ratio must be positive")
    if physical:
        _dtype(table, torch.int32, "table")
        _require(table.dim() == 2 and (table.size(1) <= 1 or table.stride(1) == 1),
                 "table must be [requests, width] with unit column stride")
        _require(page_size > 0, "page_size must be positive")
    if store_counts:
        _vector(counts, torch.int32, "counts", rows)
    if rows == 0:
        return
    width = output.size(1)
    topk = width // ratio
    lib = _lib.load()
    ws = _workspace(lib.qsa_topk_workspace_bytes(rows, cols, topk), dev)
    with torch.cuda.device(dev):
        _lib.call(
            "qsa_topk_expand", _ptr(scores), scores.stride(0), rows, cols,
            _ptr(lengths), _ptr(positions), _ptr(sequence_lengths), sequence_lengths.numel(),
            _ptr(token_to_req),
            _ptr(table if physical else None), table.stride(0) if physical else 0,
            table.size(1) if physical else 0,
            _ptr(output), output.stride(0), output.stride(1), width,
            _ptr(counts if store_counts else None), int(ratio), int(page_size),
            int(bool(physical)), int(bool(store_counts)),
            _ptr(ws), 0 if ws is None else ws.numel(), _stream(dev))


# --- indexer ----------------------------------------------------------------

# --- indexer preparation ------------------------------------------------------

def _bf16_vec(t, n, name):
    _dtype(t, torch.bfloat16, name)
    _require(t.dim() == 1 and t.numel() == n and (n <= 1 or t.stride(0) == 1),
             f"{name} must be a contiguous [{n}] vector")


def _rotary_cache(cos_sin, rotary_dim, name="cos_sin"):
    _dtype(cos_sin, torch.bfloat16, name)
    _require(cos_sin.dim() == 2 and cos_sin.size(1) == rotary_dim and cos_sin.is_contiguous(),
             f"{name} must be a contiguous [positions, rotary_dim] tensor")


def _positions(t, n, name):
    _dtype(t, torch.int64, name)
    _require(t.dim() == 1 and t.numel() >= n, f"{name} must be 1-D with at least {n} entries")


def _unit_dim(t, name, dims):
    _dtype(t, torch.bfloat16, name)
    _require(t.dim() == dims and t.stride(-1) == 1, f"{name} must be {dims}-D with unit dim stride")


def _indexer_prepare_impl(index_qk, positions, q_norm_weight, k_norm_weight, cos_sin, eps,
                          index_q_out, state_cache, state_slots, state_table, query_start_loc,
                          logical_positions, compressed_cache, compressed_slots, k_work,
                          main_key, main_value, main_key_cache, main_value_cache, main_slots,
                          num_index_heads, index_head_dim, rotary_dim, compress_ratio):
    dev = _on_gpu(index_qk, positions, q_norm_weight, k_norm_weight, cos_sin, index_q_out,
                  state_cache, state_slots, state_table, query_start_loc, logical_positions,
                  compressed_cache, compressed_slots, k_work, main_key, main_value,
                  main_key_cache, main_value_cache, main_slots)
    tokens = index_qk.size(0)
    heads, dim = int(num_index_heads), int(index_head_dim)
    _unit_dim(index_qk, "index_qk", 2)
    _require(index_qk.size(1) >= (heads + 1) * dim, "index_qk must hold (heads + 1) * dim columns")
    _positions(positions, tokens, "positions")
    _bf16_vec(q_norm_weight, dim, "q_norm_weight")
    _bf16_vec(k_norm_weight, dim, "k_norm_weight")
    _rotary_cache(cos_sin, rotary_dim)
    _dtype(index_q_out, torch.bfloat16, "index_q_out")
    _require(index_q_out.is_contiguous() and index_q_out.numel() == tokens * heads * dim,
             "index_q_out must be a contiguous [tokens, heads, dim] tensor")
    for t, name in ((state_cache, "state_cache"), (compressed_cache, "compressed_cache")):
        _dtype(t, torch.bfloat16, name)
        _require(t.dim() in (3, 4) and t.stride(-1) == 1 and t.size(-1) == dim
                 and (t.dim() == 3 or t.size(2) == 1),
                 f"{name} must be [blocks, page, (1,) dim] with unit dim stride")
    for t, name in ((state_slots, "state_slots"), (compressed_slots, "compressed_slots"),
                    (main_slots, "main_slots")):
        _positions(t, tokens, name)
        _require(t.numel() <= 1 or t.stride(0) == 1, f"{name} must be contiguous")
    _positions(logical_positions, tokens, "logical_positions")
    _require(logical_positions.numel() <= 1 or logical_positions.stride(0) == 1,
             "logical_positions must be contiguous")
    _dtype(state_table, torch.int32, "state_table")
    _require(state_table.dim() == 2, "state_table must be [requests, width]")
    _vector(query_start_loc, torch.int32, "query_start_loc")
    num_requests = query_start_loc.numel() - 1
    _require(state_table.size(0) >= num_requests, "state_table has fewer rows than requests")
    _dtype(k_work, torch.int32, "k_work")
    _require(k_work.dim() == 2 and k_work.size(1) == 2 and k_work.is_contiguous(),
             "k_work must be a contiguous [items, 2] tensor")
    _unit_dim(main_key, "main_key", 3)
    _unit_dim(main_value, "main_value", 3)
    _unit_dim(main_key_cache, "main_key_cache", 4)
    _unit_dim(main_value_cache, "main_value_cache", 4)
    kv_heads, main_dim = main_key.size(1), main_key.size(2)
    _require(tuple(main_value.shape) == (tokens, kv_heads, main_dim) and main_key.size(0) == tokens,
             "main_key / main_value must be [tokens, kv_heads, dim]")
    _require(main_key_cache.shape == main_value_cache.shape
             and main_key_cache.size(2) == kv_heads and main_key_cache.size(3) == main_dim,
             "main caches must be [blocks, page, kv_heads, dim] matching main_key")
    if tokens == 0 and k_work.size(0) == 0:
        return
    with torch.cuda.device(dev):
        _lib.call("qsa_indexer_prepare",
                  _ptr(index_qk), _stride(index_qk, 0), tokens,
                  _ptr(positions), _stride(positions, 0),
                  _ptr(q_norm_weight), _ptr(k_norm_weight),
                  _ptr(cos_sin), cos_sin.size(0), ctypes.c_float(eps),
                  _ptr(index_q_out),
                  _ptr(state_cache), _stride(state_cache, 0),
                  _stride(state_cache, 1), state_cache.size(1), state_cache.size(0),
                  _ptr(state_slots), _ptr(state_table),
                  _stride(state_table, 0), _ptr(query_start_loc),
                  _ptr(logical_positions), num_requests,
                  _ptr(compressed_cache), _stride(compressed_cache, 0),
                  _stride(compressed_cache, 1), compressed_cache.size(1), compressed_cache.size(0),
                  _ptr(compressed_slots), _ptr(k_work), k_work.size(0),
                  _ptr(main_key), _stride(main_key, 0), _stride(main_key, 1),
                  _ptr(main_value), _stride(main_value, 0), _stride(main_value, 1),
                  _ptr(main_key_cache), _stride(main_key_cache, 0), _stride(main_key_cache, 1),
                  _stride(main_key_cache, 2),
                  _ptr(main_value_cache), _stride(main_value_cache, 0),
                  _stride(main_value_cache, 1), _stride(main_value_cache, 2),
                  _ptr(main_slots), main_key_cache.size(1), main_key_cache.size(0),
                  heads, dim, int(rotary_dim), int(compress_ratio), kv_heads, main_dim,
                  _stream(dev))


def _indexer_norm_rope_impl(values, weight, positions, cos_sin, eps, rotary_dim, out):
    dev = _on_gpu(values, weight, positions, cos_sin, out)
    _unit_dim(values, "values", 3)
    tokens, heads, dim = values.shape
    _bf16_vec(weight, dim, "weight")
    _positions(positions, tokens, "positions")
    _rotary_cache(cos_sin, rotary_dim)
    _dtype(out, torch.bfloat16, "out")
    _require(out.is_contiguous() and tuple(out.shape) == (tokens, heads, dim),
             "out must be a contiguous tensor shaped like values")
    if tokens == 0 or heads == 0:
        return
    with torch.cuda.device(dev):
        _lib.call("qsa_indexer_norm_rope", _ptr(values), _stride(values, 0), _stride(values, 1),
                  tokens, heads, dim, _ptr(weight), _ptr(positions), _stride(positions, 0),
                  _ptr(cos_sin), cos_sin.size(0), ctypes.c_float(eps), int(rotary_dim),
                  _ptr(out), _stream(dev))


def _store_cache_rows_impl(cache, slot_mapping, rows):
    dev = _on_gpu(cache, slot_mapping, rows)
    _dtype(cache, torch.bfloat16, "cache")
    _require(cache.dim() == 4 and cache.stride(3) == 1, "cache must be [blocks, page, heads, width] "
             "with unit width stride")
    if rows.dim() == 3:
        rows = rows[:, 0]
    _dtype(rows, torch.bfloat16, "rows")
    _require(rows.dim() == 2 and rows.stride(1) == 1 and rows.size(1) >= cache.size(3),
             "rows must be [rows, >= width] with unit dim stride")
    _positions(slot_mapping, rows.size(0), "slot_mapping")
    _require(slot_mapping.numel() <= 1 or slot_mapping.stride(0) == 1, "slot_mapping must be contiguous")
    if rows.size(0) == 0:
        return
    with torch.cuda.device(dev):
        _lib.call("qsa_store_cache_rows", _ptr(cache), _stride(cache, 0), _stride(cache, 1),
                  cache.size(0), cache.size(1), cache.size(3), _ptr(slot_mapping), _ptr(rows),
                  _stride(rows, 0), rows.size(0), _stream(dev))


def _compress_groups_impl(raw_keys, raw_positions, state_cache, rope_cache, state_table,
                          token_to_req, query_start_loc, logical_positions, compressed_slots,
                          ratio, pooled, first_positions):
    dev = _on_gpu(raw_keys, raw_positions, state_cache, rope_cache, state_table, token_to_req,
                  query_start_loc, logical_positions, compressed_slots, pooled, first_positions)
    _dtype(raw_keys, torch.bfloat16, "raw_keys")
    _require(raw_keys.dim() == 3 and raw_keys.size(1) == 1 and raw_keys.stride(2) == 1,
             "raw_keys must be [rows, 1, dim] with unit dim stride")
    dim = raw_keys.size(2)
    _dtype(state_cache, torch.bfloat16, "compressor_state_cache")
    _require(state_cache.dim() == 4 and state_cache.size(2) == 1 and state_cache.stride(3) == 1
             and state_cache.size(3) >= dim,
             "compressor_state_cache must be [blocks, ring, 1, >= dim] with unit dim stride")
    _vector(token_to_req, torch.int32, "token_to_req")
    rows = token_to_req.numel()
    _vector(query_start_loc, torch.int32, "query_start_loc")
    _dtype(state_table, torch.int32, "compressor_state_block_table")
    _require(state_table.dim() == 2 and state_table.size(0) >= query_start_loc.numel() - 1,
             "compressor_state_block_table must be [requests, width]")
    for t, name in ((logical_positions, "logical_positions"), (compressed_slots, "compressed_slots")):
        _positions(t, rows, name)
        _require(t.numel() <= 1 or t.stride(0) == 1, f"{name} must be contiguous")
    _require(raw_keys.size(0) >= rows, "raw_keys has fewer rows than token_to_req")
    _dtype(pooled, torch.bfloat16, "pooled")
    _require(pooled.dim() == 3 and pooled.size(0) >= rows and pooled.size(2) == dim
             and pooled.stride(2) == 1, "pooled must be [rows, 1, dim]")
    _dtype(first_positions, torch.int64, "first_positions")
    _require(first_positions.dim() == 2 and first_positions.size(1) >= 3,
             "first_positions must be [rows, 3]")
    rp = (0, 0)
    if rope_cache is not None:
        _dtype(rope_cache, torch.int64, "rope_cache")
        _require(rope_cache.dim() == 4 and rope_cache.size(3) >= 3, "rope_cache must be "
                 "[blocks, ring, 1, >= 3] int64")
        _dtype(raw_positions, torch.int64, "raw_positions")
        _require(raw_positions.dim() == 3 and raw_positions.size(2) >= 3,
                 "raw_positions must be [rows, 1, >= 3] int64")
        rp = (_stride(raw_positions, 0), _stride(raw_positions, 2))
    if rows == 0:
        return
    with torch.cuda.device(dev):
        _lib.call("qsa_compress_groups", _ptr(raw_keys), _stride(raw_keys, 0),
                  _ptr(raw_positions if rope_cache is not None else None), rp[0], rp[1],
                  _ptr(state_cache), _stride(state_cache, 0), _stride(state_cache, 1),
                  state_cache.size(1), state_cache.size(0),
                  _ptr(rope_cache), _stride(rope_cache, 0) if rope_cache is not None else 0,
                  _stride(rope_cache, 1) if rope_cache is not None else 0,
                  _stride(rope_cache, 3) if rope_cache is not None else 0,
                  _ptr(state_table), _stride(state_table, 0), _ptr(token_to_req),
                  _ptr(query_start_loc), query_start_loc.numel() - 1, _ptr(logical_positions),
                  _ptr(compressed_slots), rows, dim, int(ratio), _ptr(pooled),
                  _stride(pooled, 0), _ptr(first_positions), _stride(first_positions, 0),
                  first_positions.stride(1), _stream(dev))


def _expand_block_indices_impl(block_indices, positions, sequence_lengths, token_to_req, table,
                               output, counts, ratio, topk, page_size, physical, store_counts):
    dev = _on_gpu(block_indices, positions, sequence_lengths, token_to_req, table, output, counts)
    _dtype(block_indices, torch.int32, "block_indices")
    _require(block_indices.dim() == 2, "block_indices must be [rows, blocks]")
    rows = block_indices.size(0)
    _positions(positions, rows, "query_positions")
    _vector(sequence_lengths, torch.int32, "sequence_lengths")
    _vector(token_to_req, torch.int32, "token_to_req", rows)
    _dtype(output, torch.int32, "output")
    _require(output.dim() == 2 and output.size(0) >= rows, "output must be [rows, width]")
    if physical:
        _dtype(table, torch.int32, "main_block_table")
        _require(table.dim() == 2 and (table.size(1) <= 1 or table.stride(1) == 1),
                 "main_block_table must be [requests, width] with unit column stride")
    if store_counts:
        _vector(counts, torch.int32, "valid_counts_out", rows)
    if rows == 0:
        return
    with torch.cuda.device(dev):
        _lib.call("qsa_expand_block_indices", _ptr(block_indices), _stride(block_indices, 0),
                  _stride(block_indices, 1), block_indices.size(1), rows, int(topk),
                  _ptr(positions), _ptr(sequence_lengths), sequence_lengths.numel(),
                  _ptr(token_to_req), _ptr(table if physical else None),
                  table.stride(0) if physical else 0, table.size(1) if physical else 0,
                  _ptr(output), _stride(output, 0), output.stride(1), output.size(1),
                  _ptr(counts if store_counts else None), int(ratio), int(page_size),
                  1 if physical else 0, 1 if store_counts else 0, _stream(dev))


def _cache_strides(k_cache, name):
    _dtype(k_cache, torch.bfloat16, name)
    _require(k_cache.dim() in (3, 4), f"{name} must be [blocks, page, (1,) dim]")
    if k_cache.dim() == 4:
        _require(k_cache.size(2) == 1, f"{name} must hold one index head")
    _require(k_cache.stride(-1) == 1, f"{name} must have a unit dim stride")
    return _stride(k_cache, 0), _stride(k_cache, 1)


def _indexer_decode_impl(q, k_cache, page_table, visible, logits, decode_query_len):
    dev = _on_gpu(q, k_cache, page_table, visible, logits)
    _dtype(q, torch.bfloat16, "q")
    _require(q.dim() == 3 and q.stride(2) == 1, "q must be [rows, heads, dim] with unit dim stride")
    rows, heads, dim = q.shape
    cb, ct = _cache_strides(k_cache, "k_cache")
    _require(k_cache.size(-1) == dim, "k_cache dim must match q")
    _dtype(page_table, torch.int32, "page_table")
    _require(page_table.dim() == 2 and (page_table.size(1) <= 1 or page_table.stride(1) == 1),
             "page_table must be [requests, width] with unit column stride")
    _vector(visible, torch.int32, "visible", rows)
    _dtype(logits, torch.float32, "logits")
    _require(logits.dim() == 2 and logits.size(0) >= rows
             and (logits.size(1) <= 1 or logits.stride(1) == 1),
             "logits must be [rows, cols] with unit column stride")
    _require(decode_query_len > 0 and page_table.size(0) * decode_query_len >= rows,
             "page_table has fewer requests than rows / decode_query_len")
    if rows == 0:
        return
    with torch.cuda.device(dev):
        _lib.call("qsa_indexer_decode", _ptr(q), _stride(q, 0), _stride(q, 1), rows, heads, dim,
                  _ptr(k_cache), cb, ct, k_cache.size(0), k_cache.size(1),
                  _ptr(page_table), page_table.stride(0), page_table.size(1),
                  _ptr(visible), int(decode_query_len), _ptr(logits), logits.stride(0),
                  logits.size(1), _stream(dev))


def _indexer_prefill_impl(q, k_cache, page_table, query_start_loc, visible, logits,
                          query_offset, num_rows, max_query_len):
    dev = _on_gpu(q, k_cache, page_table, query_start_loc, visible, logits)
    _dtype(q, torch.bfloat16, "q")
    _require(q.dim() == 3 and q.stride(2) == 1, "q must be [rows, heads, dim] with unit dim stride")
    _, heads, dim = q.shape
    cb, ct = _cache_strides(k_cache, "k_cache")
    _require(k_cache.size(-1) == dim, "k_cache dim must match q")
    _dtype(page_table, torch.int32, "page_table")
    _require(page_table.dim() == 2 and (page_table.size(1) <= 1 or page_table.stride(1) == 1),
             "page_table must be [requests, width] with unit column stride")
    requests = page_table.size(0)
    _vector(query_start_loc, torch.int32, "query_start_loc", requests + 1)
    _vector(visible, torch.int32, "visible", query_offset + num_rows)
    _require(query_offset >= 0 and q.size(0) >= query_offset + num_rows,
             "q has fewer rows than query_offset + num_rows")
    _dtype(logits, torch.float32, "logits")
    _require(logits.dim() == 2 and logits.size(0) >= num_rows
             and (logits.size(1) <= 1 or logits.stride(1) == 1),
             "logits must be [rows, cols] with unit column stride")
    if num_rows == 0 or requests == 0:
        return
    with torch.cuda.device(dev):
        _lib.call("qsa_indexer_prefill", _ptr(q), _stride(q, 0), _stride(q, 1), heads, dim,
                  _ptr(k_cache), cb, ct, k_cache.size(0), k_cache.size(1),
                  _ptr(page_table), page_table.stride(0), page_table.size(1), requests,
                  _ptr(query_start_loc), _ptr(visible), int(query_offset), int(num_rows),
                  int(max_query_len), _ptr(logits), logits.stride(0), logits.size(1),
                  _stream(dev))


# --- sparse attention ---------------------------------------------------------

def _gate_strides(gate, rows, heads, dim):
    if gate is None:
        return 0, 0, 0
    _dtype(gate, torch.bfloat16, "output_gate")
    _require(gate.dim() == 3 and tuple(gate.shape[1:]) == (heads, dim) and gate.size(0) >= rows,
             "output_gate must be [rows, heads, dim]")
    return _stride(gate, 0), _stride(gate, 1), _stride(gate, 2)


def _sparse_attention_impl(q, k_cache, v_cache, indices, block_table, token_to_req, out,
                           output_gate, valid_counts, indices_are_physical, num_splits):
    dev = _on_gpu(q, k_cache, v_cache, indices, block_table, token_to_req, out, output_gate,
                  valid_counts)
    for t, name in ((q, "q"), (k_cache, "k_cache"), (v_cache, "v_cache"), (out, "out")):
        _dtype(t, torch.bfloat16, name)
    _require(q.dim() == 3 and q.stride(2) == 1, "q must be [rows, heads, dim] with unit dim stride")
    rows, hq, dim = q.shape
    _require(k_cache.dim() == 4 and v_cache.dim() == 4 and k_cache.shape == v_cache.shape,
             "k_cache/v_cache must be [blocks, page, kv_heads, dim] of one shape")
    _require(k_cache.stride(3) == 1 and v_cache.stride(3) == 1, "k/v caches need a unit dim stride")
    _require(k_cache.size(3) == dim, "cache head dim must match q")
    _require(out.dim() == 3 and tuple(out.shape[1:]) == (hq, dim) and out.size(0) >= rows
             and out.stride(2) == 1, "out must be [rows, heads, dim] with unit dim stride")
    _dtype(indices, torch.int32, "indices")
    _require(indices.dim() == 2 and indices.size(0) >= rows
             and (indices.size(1) <= 1 or indices.stride(1) == 1),
             "indices must be [rows, width] with unit column stride")
    _dtype(block_table, torch.int32, "block_table")
    _require(block_table.dim() == 2 and (block_table.size(1) <= 1 or block_table.stride(1) == 1),
             "block_table must be [requests, width] with unit column stride")
    _vector(token_to_req, torch.int32, "token_to_req", rows)
    if valid_counts is not None:
        _vector(valid_counts, torch.int32, "valid_counts", rows)
    gr, gh, gd = _gate_strides(output_gate, rows, hq, dim)
    if rows == 0:
        return
    lib = _lib.load()
    nbytes = lib.qsa_sparse_attention_workspace_bytes(rows, hq, dim, int(num_splits))
    ws = _workspace(nbytes, dev)
    with torch.cuda.device(dev):
        _lib.call(
            "qsa_sparse_attention", _ptr(q), _stride(q, 0), _stride(q, 1), rows, hq, dim,
            _ptr(k_cache), _stride(k_cache, 0), _stride(k_cache, 1), _stride(k_cache, 2),
            _ptr(v_cache), _stride(v_cache, 0), _stride(v_cache, 1), _stride(v_cache, 2),
            k_cache.size(0), k_cache.size(1), k_cache.size(2),
            _ptr(indices), indices.stride(0), indices.size(1),
            _ptr(block_table), block_table.stride(0), block_table.size(1), block_table.size(0),
            _ptr(token_to_req), _ptr(valid_counts),
            _ptr(out), _stride(out, 0), _stride(out, 1),
            _ptr(output_gate), gr, gh, gd,
            int(bool(indices_are_physical)), int(num_splits),
            _ptr(ws), 0 if ws is None else ws.numel(), _stream(dev))


def _sparse_attention_merge_impl(partial_out, partial_lse, out, output_gate):
    dev = _on_gpu(partial_out, partial_lse, out, output_gate)
    _dtype(partial_out, torch.float32, "partial_out")
    _dtype(partial_lse, torch.float32, "partial_lse")
    _dtype(out, torch.bfloat16, "out")
    _require(partial_out.dim() == 4 and partial_out.is_contiguous(),
             "partial_out must be contiguous [splits, rows, heads, dim]")
    splits, rows, hq, dim = partial_out.shape
    _require(partial_lse.shape == (splits, rows, hq) and partial_lse.is_contiguous(),
             "partial_lse must be contiguous [splits, rows, heads]")
    _require(out.dim() == 3 and tuple(out.shape[1:]) == (hq, dim) and out.size(0) >= rows
             and out.stride(2) == 1, "out must be [rows, heads, dim] with unit dim stride")
    gr, gh, gd = _gate_strides(output_gate, rows, hq, dim)
    if rows == 0:
        return
    with torch.cuda.device(dev):
        _lib.call("qsa_sparse_attention_merge", _ptr(partial_out), _ptr(partial_lse), splits,
                  rows, hq, dim, _ptr(out), _stride(out, 0), _stride(out, 1), _ptr(output_gate),
                  gr, gh, gd, _stream(dev))


_IMPLS = {
    "topk": _topk_impl,
    "topk_expand": _topk_expand_impl,
    "indexer_decode": _indexer_decode_impl,
    "indexer_prefill": _indexer_prefill_impl,
    "sparse_attention": _sparse_attention_impl,
    "sparse_attention_merge": _sparse_attention_merge_impl,
    "indexer_prepare": _indexer_prepare_impl,
    "indexer_norm_rope": _indexer_norm_rope_impl,
    "store_cache_rows": _store_cache_rows_impl,
    "compress_groups": _compress_groups_impl,
    "expand_block_indices": _expand_block_indices_impl,
}

_library = None


def register() -> None:
    """Define the ops (once per process) with a CUDA-key kernel and a no-op Meta kernel."""
    global _library
    if _library is not None:
        return
    lib = torch.library.Library(_NS, "FRAGMENT")
    for name, schema in _SCHEMAS.items():
        lib.define(schema)
        lib.impl(name, _IMPLS[name], "CUDA")
        lib.impl(name, lambda *args, **kwargs: None, "Meta")
    _library = lib


register()
