"""Index-key scoring and top-k token selection (host side of the QSA indexer).

The entry points keep the names, arguments and results of the reference
``yulan_qsa_vllm/ops/indexer.py``: ``qsa_select_paged_decode`` (:227-239),
``qsa_select_paged_prefill`` (:305-318) and ``select_paged_tokens``
(:346-393). Each call scores queries into an fp32 logits buffer with the HIP
scoring kernel and then runs the fused top-k + expansion kernel on it, all
inside one op (``select_decode`` / ``select_prefill``), so the host pays one
dispatcher call per selection.

The logits buffer is capped at ``QSA_INDEXER_WORKSPACE_MB`` MiB (default 64,
the reference's cap); a call whose rows need more is processed in row spans
that each fit, reusing the one buffer. Spans only bound memory: every row's
result is independent of how the rows are grouped.
"""

from __future__ import annotations

import os

import torch

from ..graph_dispatch import decode_logits_columns, prefill_logits_width

_LOGITS_CAP_BYTES = int(os.environ.get("QSA_INDEXER_WORKSPACE_MB", "64")) << 20


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
    ``[i * decode_query_len, (i + 1) * decode_query_len)`` of ``q``. Logits
    take the decode width class; spans of whole requests keep the buffer
    within the cap (``ops/indexer.py:245-252``)."""
    columns = decode_logits_columns(max_seq_len, compress_ratio,
                                    page_table.shape[1] * k_cache.shape[1])
    torch.ops.yulan_qsa_kernels.select_decode(
        q, k_cache, page_table, visible_blocks, query_positions, sequence_lengths, token_to_req,
        out, main_block_table, valid_counts_out, compress_ratio, decode_query_len, columns,
        main_page_size, _LOGITS_CAP_BYTES)


def decode_select_attend(
    index_q: torch.Tensor,
    index_cache: torch.Tensor,
    index_table: torch.Tensor,
    visible_blocks: torch.Tensor,
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    main_block_table: torch.Tensor,
    token_to_req: torch.Tensor,
    query_positions: torch.Tensor,
    sequence_lengths: torch.Tensor,
    token_topk: int,
    compress_ratio: int,
    max_seq_len: int,
    indices_out: torch.Tensor,
    counts_out: torch.Tensor,
    out: torch.Tensor,
    *,
    output_gate: torch.Tensor | None = None,
    num_splits: int = 0,
) -> torch.Tensor:
    """A decode batch (one row per request) from index queries to attention
    output: the selection of :func:`qsa_select_paged_decode` with physical
    slots (``indices_out``, ``counts_out``) and the backend's sparse attention
    over it (``qsa_sparse_paged_attention`` with ``indices_are_physical`` and
    ``valid_counts``; ``backend.py:49-68``), same results. The scores go to a
    logits buffer of the decode width class; the top-k, expansion and
    attention then run as one op, which launches them as one kernel (plus the
    split merge) for the batch shapes the library fuses. ``num_splits`` 0 is
    the library's split choice. Batches whose logits exceed the workspace cap
    run the two calls."""
    rows = index_q.shape[0]
    if rows == 0:
        return out
    columns = decode_logits_columns(max_seq_len, compress_ratio,
                                    index_table.shape[1] * index_cache.shape[1])
    if rows * columns * 4 > _LOGITS_CAP_BYTES:
        qsa_select_paged_decode(index_q, index_cache, index_table, visible_blocks, token_topk,
                                compress_ratio, 1, indices_out, max_seq_len,
                                query_positions=query_positions,
                                sequence_lengths=sequence_lengths, token_to_req=token_to_req,
                                main_block_table=main_block_table,
                                main_page_size=k_cache.shape[1], valid_counts_out=counts_out)
        torch.ops.yulan_qsa_kernels.sparse_attention(
            q, k_cache, v_cache, indices_out, main_block_table, token_to_req, out, output_gate,
            counts_out, True, int(num_splits))
        return out
    logits = torch.empty(rows, columns, dtype=torch.float32, device=index_q.device)
    torch.ops.yulan_qsa_kernels.indexer_decode(index_q, index_cache, index_table, visible_blocks,
                                               logits, 1)
    torch.ops.yulan_qsa_kernels.decode_select_attend(
        logits, visible_blocks, query_positions, sequence_lengths, token_to_req, main_block_table,
        indices_out, counts_out, compress_ratio, q, k_cache, v_cache, out, output_gate,
        int(num_splits))
    return out


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
    its ``visible_blocks`` entry. Spans stay within the cap; the library
    rounds them to whole launch rounds (only the launch count differs from
    the reference's chunks, ``ops/indexer.py:324-329``)."""
    width = prefill_logits_width(max_seq_len, compress_ratio,
                                 page_table.shape[1] * k_cache.shape[1])
    torch.ops.yulan_qsa_kernels.select_prefill(
        q, k_cache, page_table, query_start_loc, visible_blocks, query_positions,
        sequence_lengths, token_to_req, out, main_block_table, valid_counts_out, compress_ratio,
        max_query_len, width, main_page_size, _LOGITS_CAP_BYTES)


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

    def part(t, rows: slice):
        # a whole-batch part takes the caller's tensors as they are
        return t if t is None or (rows.start == 0 and rows.stop == rows_total) else t[rows]

    def row_args(rows: slice):
        return dict(
            query_positions=part(query_positions, rows), sequence_lengths=sequence_lengths,
            token_to_req=part(token_to_req, rows), main_block_table=main_block_table,
            main_page_size=main_page_size, valid_counts_out=part(valid_counts_out, rows))

    split = num_decode_tokens
    if split > 0:
        rows = slice(0, split)
        qsa_select_paged_decode(part(q, rows), k_cache, page_table[:num_decodes],
                                part(visible_blocks, rows), token_topk, compress_ratio,
                                decode_query_len, part(out, rows), max_seq_len, **row_args(rows))
    if split < rows_total:
        rows = slice(split, rows_total)
        qsa_select_paged_prefill(part(q, rows), k_cache, page_table[num_decodes:],
                                 query_start_loc[num_decodes:], part(visible_blocks, rows),
                                 token_topk, compress_ratio, max_query_len, part(out, rows),
                                 max_seq_len, **row_args(rows))
    return out
