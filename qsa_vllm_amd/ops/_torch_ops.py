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
