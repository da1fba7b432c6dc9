"""QSA indexer scoring + fused top-k selection on gfx950.

Same functions, signatures and chunking policy as the reference
``yulan_qsa_vllm/ops/indexer.py``: ``qsa_select_paged_decode`` (:227-279),
``qsa_select_paged_prefill`` (:305-343), ``select_paged_tokens`` (:346-393).
Scoring runs in the HIP kernels behind ``torch.ops.yulan_qsa_kernels.
indexer_decode`` / ``indexer_prefill`` and selection in ``topk_expand``. The
fp32 logits workspace is bounded by ``QSA_INDEXER_WORKSPACE_MB`` (default 64),
as in the reference.
"""

from __future__ import annotations

import os

import torch

from ..graph_dispatch import decode_logits_columns
from .topk import topk_expand as _topk_expand

_INDEXER_WORKSPACE_BYTES = int(os.environ.get("QSA_INDEXER_WORKSPACE_MB", "64")) * 1024 * 1024


def _cdiv(a: int, b: int) -> int:
    return (a + b - 1) // b


def qsa_select_paged_decode(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    page_table: torch.Tensor,
    visible_blocks: torch.Tensor,
    token_topk: int,
    compress_ratio: int,
    decode_query_len: int,
    out: torch.Tensor,
    max_seq_len: int,
    *, query_positions, sequence_lengths, token_to_req,
    main_block_table=None, main_page_size=1, valid_counts_out=None,
) -> None:
    """Score decode queries and write the expanded selection."""
    num_requests = q.shape[0] // decode_query_len
    columns = decode_logits_columns(
        max_seq_len, compress_ratio, page_table.shape[1] * k_cache.shape[1],
    )
    requests_per_chunk = max(
        1, _INDEXER_WORKSPACE_BYTES // (columns * 4 * decode_query_len)
    )
    workspace_rows = min(num_requests, requests_per_chunk) * decode_query_len
    logits_workspace = torch.empty(
        (workspace_rows, columns), dtype=torch.float32, device=q.device,
    )
    for first_request in range(0, num_requests, requests_per_chunk):
        last_request = min(first_request + requests_per_chunk, num_requests)
        first_row = first_request * decode_query_len
        last_row = last_request * decode_query_len
        queries = q[first_row:last_row]
        table = page_table[first_request:last_request]
        visible = visible_blocks[first_row:last_row]
        logits = logits_workspace[:last_row - first_row]
        torch.ops.yulan_qsa_kernels.indexer_decode(
            queries, k_cache, table, visible, logits, decode_query_len)
        _topk_expand(
            logits, visible, query_positions[first_row:last_row], sequence_lengths,
            token_to_req[first_row:last_row], out[first_row:last_row], compress_ratio,
            main_block_table=main_block_table, main_page_size=main_page_size,
            valid_counts_out=(valid_counts_out[first_row:last_row]
                              if valid_counts_out is not None else None),
        )


def _prefill_logits(
    q, k_cache, page_table, query_start_loc, visible_blocks, logits_workspace,
    max_query_len, logits_width, query_offset, num_queries,
):
    logits = logits_workspace[:num_queries * logits_width].view(num_queries, logits_width)
    torch.ops.yulan_qsa_kernels.indexer_prefill(
        q, k_cache, page_table, query_start_loc, visible_blocks, logits,
        query_offset, num_queries, max_query_len)
    return logits


def qsa_select_paged_prefill(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    page_table: torch.Tensor,
    query_start_loc: torch.Tensor,
    visible_blocks: torch.Tensor,
    token_topk: int,
    compress_ratio: int,
    max_query_len: int,
    out: torch.Tensor,
    max_seq_len: int,
    *, query_positions, sequence_lengths, token_to_req,
    main_block_table=None, main_page_size=1, valid_counts_out=None,
) -> None:
    """Packed prefill scoring and fused final token-selection writeout."""
    rows = q.shape[0]
    columns = page_table.shape[1] * k_cache.shape[1]
    logits_width = _cdiv(_cdiv(max_seq_len, compress_ratio), 64) * 64
    logits_width = min(max(64, logits_width), columns)
    rows_per_chunk = max(1, _INDEXER_WORKSPACE_BYTES // (logits_width * 4))
    logits_workspace = torch.empty(
        min(rows, rows_per_chunk) * logits_width,
        dtype=torch.float32, device=q.device,
    )
    for query_start in range(0, rows, rows_per_chunk):
        query_end = min(query_start + rows_per_chunk, rows)
        logits = _prefill_logits(
            q, k_cache, page_table, query_start_loc, visible_blocks,
            logits_workspace, max_query_len, logits_width,
            query_offset=query_start, num_queries=query_end - query_start,
        )
        _topk_expand(
            logits, visible_blocks[query_start:query_end],
            query_positions[query_start:query_end], sequence_lengths,
            token_to_req[query_start:query_end], out[query_start:query_end], compress_ratio,
            main_block_table=main_block_table, main_page_size=main_page_size,
            valid_counts_out=(valid_counts_out[query_start:query_end]
                              if valid_counts_out is not None else None),
        )


def select_paged_tokens(
    q, k_cache, page_table, token_to_req, query_positions, sequence_lengths,
    token_topk, compress_ratio, out=None, *, query_start_loc, max_query_len,
    max_seq_len, num_decodes=0, num_decode_tokens=0, decode_query_len=1,
    visible_blocks=None, main_block_table=None, main_page_size=1,
    valid_counts_out=None,
):
    """Select blocks and write expanded decode/prefill tokens in place."""
    rows = q.shape[0]
    if out is None:
        out = torch.empty(
            (rows, token_topk + compress_ratio - 1),
            dtype=torch.int32, device=q.device,
        )
    if not rows:
        return out
    if visible_blocks is None:
        safe_requests = token_to_req.clamp_min(0).long()
        visible_blocks = torch.minimum(
            (query_positions + 1) // compress_ratio,
            sequence_lengths.index_select(0, safe_requests) // compress_ratio,
        ).to(torch.int32)
        visible_blocks = torch.where(token_to_req >= 0, visible_blocks, 0)
    if num_decode_tokens:
        qsa_select_paged_decode(
            q[:num_decode_tokens], k_cache, page_table[:num_decodes],
            visible_blocks[:num_decode_tokens], token_topk, compress_ratio,
            decode_query_len, out[:num_decode_tokens], max_seq_len,
            query_positions=query_positions[:num_decode_tokens],
            sequence_lengths=sequence_lengths, token_to_req=token_to_req[:num_decode_tokens],
            main_block_table=main_block_table, main_page_size=main_page_size,
            valid_counts_out=(valid_counts_out[:num_decode_tokens]
                              if valid_counts_out is not None else None),
        )
    if num_decode_tokens < rows:
        qsa_select_paged_prefill(
            q[num_decode_tokens:], k_cache, page_table[num_decodes:],
            query_start_loc[num_decodes:], visible_blocks[num_decode_tokens:],
            token_topk, compress_ratio, max_query_len,
            out[num_decode_tokens:], max_seq_len,
            query_positions=query_positions[num_decode_tokens:],
            sequence_lengths=sequence_lengths, token_to_req=token_to_req[num_decode_tokens:],
            main_block_table=main_block_table, main_page_size=main_page_size,
            valid_counts_out=(valid_counts_out[num_decode_tokens:]
                              if valid_counts_out is not None else None),
        )
    return out
