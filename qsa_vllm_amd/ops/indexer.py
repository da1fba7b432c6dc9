"""Index-key scoring and top-k token selection (host side of the QSA indexer).

The entry points keep the names, arguments and results of the reference
``yulan_qsa_vllm/ops/indexer.py``: ``qsa_select_paged_decode`` (:227-239),
``qsa_select_paged_prefill`` (:305-318) and ``select_paged_tokens``
(:346-393). Each call scores queries into an fp32 logits buffer with the HIP
scoring kernel (``indexer_decode`` / ``indexer_prefill``) and then runs the
fused top-k + expansion kernel (``topk_expand``) on it.

The logits buffer is capped at ``QSA_INDEXER_WORKSPACE_MB`` MiB (default 64,
the reference's cap); a call whose rows need more is processed in row spans
that each fit, reusing the one buffer. Spans only bound memory: every row's
result is independent of how the rows are grouped.
"""

from __future__ import annotations

import os

import torch

from .. import _lib
from ..graph_dispatch import decode_logits_columns, prefill_logits_width
from .topk import topk_expand

_LOGITS_CAP_BYTES = int(os.environ.get("QSA_INDEXER_WORKSPACE_MB", "64")) << 20


def _spans(count: int, per_span: int):
    """[start, end) spans of at most ``per_span`` covering ``range(count)``."""
    return [(a, min(a + per_span, count)) for a in range(0, count, per_span)]


def _expand_rows(logits, rows: slice, visible_blocks, compress_ratio, out, *, query_positions,
                 sequence_lengths, token_to_req, main_block_table, main_page_size,
                 valid_counts_out):
    """``topk_expand`` of the logits of ``rows`` (row-relative to the caller's tensors)."""
    topk_expand(logits, visible_blocks[rows], query_positions[rows], sequence_lengths,
                token_to_req[rows], out[rows], compress_ratio,
                main_block_table=main_block_table, main_page_size=main_page_size,
                valid_counts_out=None if valid_counts_out is None else valid_counts_out[rows])


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
    """Decode selection: request i of ``page_table`` owns rows
    ``[i * decode_query_len, (i + 1) * decode_query_len)`` of ``q``."""
    per_req = decode_query_len
    requests = q.shape[0] // per_req
    columns = decode_logits_columns(max_seq_len, compress_ratio,
                                    page_table.shape[1] * k_cache.shape[1])
    reqs_per_span = max(1, _LOGITS_CAP_BYTES // (4 * columns * per_req))
    buf = torch.empty(min(requests, reqs_per_span) * per_req, columns, dtype=torch.float32,
                      device=q.device)
    for r0, r1 in _spans(requests, reqs_per_span):
        rows = slice(r0 * per_req, r1 * per_req)
        logits = buf[:(r1 - r0) * per_req]
        torch.ops.yulan_qsa_kernels.indexer_decode(
            q[rows], k_cache, page_table[r0:r1], visible_blocks[rows], logits, per_req)
        _expand_rows(logits, rows, visible_blocks, compress_ratio, out,
                     query_positions=query_positions, sequence_lengths=sequence_lengths,
                     token_to_req=token_to_req, main_block_table=main_block_table,
                     main_page_size=main_page_size, valid_counts_out=valid_counts_out)


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
    """Prefill selection: the rows of ``q`` are the packed query tokens of the
    requests of ``page_table``, request i's starting at row
    ``query_start_loc[i] - query_start_loc[0]``, each row masked causally by
    its ``visible_blocks`` entry."""
    rows_total = q.shape[0]
    width = prefill_logits_width(max_seq_len, compress_ratio,
                                 page_table.shape[1] * k_cache.shape[1])
    # Spans stay within the cap; the library rounds them to whole launch
    # rounds (only the launch count differs from the reference's chunks).
    rows_per_span = max(1, int(_lib.load().qsa_indexer_prefill_span_rows(width, _LOGITS_CAP_BYTES)))
    buf = torch.empty(min(rows_total, rows_per_span), width, dtype=torch.float32,
                      device=q.device)
    for a, b in _spans(rows_total, rows_per_span):
        logits = buf[:b - a]
        torch.ops.yulan_qsa_kernels.indexer_prefill(
            q, k_cache, page_table, query_start_loc, visible_blocks, logits, a, b - a,
            max_query_len)
        _expand_rows(logits, slice(a, b), visible_blocks, compress_ratio, out,
                     query_positions=query_positions, sequence_lengths=sequence_lengths,
                     token_to_req=token_to_req, main_block_table=main_block_table,
                     main_page_size=main_page_size, valid_counts_out=valid_counts_out)


def _visible_blocks(query_positions, sequence_lengths, token_to_req, compress_ratio):
    """Complete compressed blocks a row may see: min((pos + 1) // R,
    seq_len // R) of its request, 0 for padding rows (request < 0)."""
    req = token_to_req.long()
    has_req = req >= 0
    seq = sequence_lengths.index_select(0, req.clamp_min(0))
    vis = torch.minimum((query_positions + 1) // compress_ratio, seq // compress_ratio)
    return torch.where(has_req, vis, torch.zeros_like(vis)).to(torch.int32)


def select_paged_tokens(
    q, k_cache, page_table, token_to_req, query_positions, sequence_lengths,
    token_topk, compress_ratio, out=None, *, query_start_loc, max_query_len,
    max_seq_len, num_decodes=0, num_decode_tokens=0, decode_query_len=1,
    visible_blocks=None, main_block_table=None, main_page_size=1,
    valid_counts_out=None,
):
    """Select ``token_topk`` tokens (+ causal tail) per query row into ``out``
    ([rows, token_topk + compress_ratio - 1] int32, allocated if absent).

    Rows come decode first: the first ``num_decode_tokens`` rows belong to the
    first ``num_decodes`` requests and take the decode scorer; the remaining
    rows (requests ``num_decodes`` onward) take the prefill scorer. With
    ``main_block_table`` the selection is written as physical cache slots.
    """
    rows_total = q.shape[0]
    if out is None:
        out = torch.empty(rows_total, token_topk + compress_ratio - 1, dtype=torch.int32,
                          device=q.device)
    if rows_total == 0:
        return out
    if visible_blocks is None:
        visible_blocks = _visible_blocks(query_positions, sequence_lengths, token_to_req,
                                         compress_ratio)

    def row_args(rows: slice):
        return dict(
            query_positions=query_positions[rows], sequence_lengths=sequence_lengths,
            token_to_req=token_to_req[rows], main_block_table=main_block_table,
            main_page_size=main_page_size,
            valid_counts_out=None if valid_counts_out is None else valid_counts_out[rows])

    split = num_decode_tokens
    if split > 0:
        rows = slice(0, split)
        qsa_select_paged_decode(q[rows], k_cache, page_table[:num_decodes],
                                visible_blocks[rows], token_topk, compress_ratio,
                                decode_query_len, out[rows], max_seq_len, **row_args(rows))
    if split < rows_total:
        rows = slice(split, rows_total)
        qsa_select_paged_prefill(q[rows], k_cache, page_table[num_decodes:],
                                 query_start_loc[num_decodes:], visible_blocks[rows],
                                 token_topk, compress_ratio, max_query_len, out[rows],
                                 max_seq_len, **row_args(rows))
    return out
