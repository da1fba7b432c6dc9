"""BF16 paged sparse GQA attention on gfx950.

Same entry points and signatures as the reference ``yulan_qsa_vllm/ops/qsa.py``:
``qsa_sparse_paged_attention`` (:594-688) and ``qsa_select_paged_tokens``
(:753-782), plus the module's helpers that nothing in the plugin calls:
``expand_qsa_block_indices_cuda`` (:552-591), ``qsa_store_cache_rows``
(:691-706) and ``qsa_compress_groups_with_ratio`` (:709-750). The split-K
kernel and the LSE merge run in ``libqsa_hip.so`` behind
``torch.ops.yulan_qsa_kernels.sparse_attention``; the helpers behind
``expand_block_indices``, ``store_cache_rows`` and ``compress_groups``.

``decode_config`` keeps the reference's ``(block_n, target_splits, warps)``
tuple and, as there, applies to the decode kernel only (``use_decode_kernel``;
``ops/qsa.py:620-622``). The split count follows the reference's rule from the
caller's ``block_n`` and ``target_splits``:
``num_splits = min(pow2floor(cdiv(W, block_n)), target_splits)``
(``ops/qsa.py:643-645``), at least 1 and at most 1024 (the library's bound;
the result does not depend on the split count beyond fp32 rounding). ``warps``
has no effect: the HIP kernel walks fixed 32-token tiles whatever ``block_n``
says and chooses its own waves per workgroup from the launch shape.
"""

from __future__ import annotations

import torch

from .. import _lib
from .topk import _torch_ops  # noqa: F401  (registers torch.ops.yulan_qsa_kernels)

_MAX_SPLITS = 1024


def _pow2floor(x: int) -> int:
    return 1 << (max(1, x).bit_length() - 1)


def config_num_splits(width: int, decode_config) -> int:
    """The reference's split count for a caller's ``(block_n, target_splits,
    warps)`` (``ops/qsa.py:643-645``): ``min(pow2floor(cdiv(width, block_n)),
    target_splits)``, clamped to [1, 1024]."""
    block_n, target = int(decode_config[0]), int(decode_config[1])
    if block_n <= 0:
        raise ValueError(f"decode_config block_n must be positive, got {block_n}")
    tiles = -(-int(width) // block_n)
    return max(1, min(_pow2floor(tiles), target, _MAX_SPLITS))


def choose_num_splits(q, k_cache, logical_indices, use_decode_kernel, decode_config=None):
    """Split count for a call: the caller's ``decode_config`` on the decode
    kernel, else the library's choice for the shape."""
    rows, hq, dim = q.shape
    width = logical_indices.shape[1]
    if use_decode_kernel and decode_config is not None:
        return config_num_splits(width, decode_config)
    return _lib.load().qsa_sparse_attention_splits(
        rows, hq, k_cache.shape[2], dim, width, int(bool(use_decode_kernel)))


def qsa_sparse_paged_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    logical_indices: torch.Tensor,
    block_table: torch.Tensor,
    token_to_req: torch.Tensor,
    out: torch.Tensor | None = None,
    *,
    output_gate: torch.Tensor | None = None,
    use_decode_kernel: bool = False,
    indices_are_physical: bool = False,
    valid_counts: torch.Tensor | None = None,
    decode_config: tuple[int, int, int] | None = None,
) -> torch.Tensor:
    """BF16 paged GQA over the selected slots (physical decode or logical prefill)."""
    if out is None:
        out = torch.empty_like(q)
    if not q.shape[0]:
        return out
    uses_config = bool(use_decode_kernel) and decode_config is not None
    if not uses_config and bool(use_decode_kernel) == bool(indices_are_physical):
        num_splits = 0  # the library's choice for this shape, made inside the op
    else:
        num_splits = choose_num_splits(q, k_cache, logical_indices, use_decode_kernel,
                                       decode_config)
    torch.ops.yulan_qsa_kernels.sparse_attention(
        q, k_cache, v_cache, logical_indices, block_table, token_to_req, out,
        output_gate, valid_counts, bool(indices_are_physical), int(num_splits))
    return out


def qsa_select_paged_tokens(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    page_table: torch.Tensor,
    token_to_req: torch.Tensor,
    query_positions: torch.Tensor,
    sequence_lengths: torch.Tensor,
    token_topk: int,
    compress_ratio: int,
    out: torch.Tensor | None = None,
    *,
    query_start_loc: torch.Tensor,
    max_query_len: int,
    max_seq_len: int,
    num_decodes: int = 0,
    num_decode_tokens: int = 0,
    decode_query_len: int = 1,
    visible_blocks: torch.Tensor | None = None,
) -> torch.Tensor:
    """Entry point of the same name in the reference's ``ops/qsa.py``
    (:753-782): :func:`select_paged_tokens` without the main-table (physical
    slot) and valid-count arguments, i.e. logical token ids."""
    from .indexer import select_paged_tokens

    return select_paged_tokens(
        q, k_cache, page_table, token_to_req, query_positions, sequence_lengths,
        token_topk, compress_ratio, out,
        query_start_loc=query_start_loc, max_query_len=max_query_len,
        max_seq_len=max_seq_len, num_decodes=num_decodes,
        num_decode_tokens=num_decode_tokens, decode_query_len=decode_query_len,
        visible_blocks=visible_blocks,
    )


def expand_qsa_block_indices_cuda(
    block_indices: torch.Tensor,
    query_positions: torch.Tensor,
    sequence_lengths: torch.Tensor,
    token_to_req: torch.Tensor,
    compress_ratio: int,
    token_topk: int,
    out: torch.Tensor | None = None,
    *,
    main_block_table: torch.Tensor | None = None,
    main_page_size: int = 1,
    valid_counts_out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Expand caller-chosen complete blocks (rank i = column i of
    ``block_indices``) plus the visible causal tail into token ids or, with
    ``main_block_table``, physical slots (ops/qsa.py:552-591)."""
    output_width = token_topk + compress_ratio - 1
    if out is None:
        out = torch.empty((block_indices.shape[0], output_width), dtype=torch.int32,
                          device=block_indices.device)
    if not block_indices.shape[0]:
        return out
    physical = main_block_table is not None
    torch.ops.yulan_qsa_kernels.expand_block_indices(
        block_indices, query_positions, sequence_lengths, token_to_req,
        main_block_table if physical else out, out,
        valid_counts_out if valid_counts_out is not None else out,
        int(compress_ratio), int(token_topk // compress_ratio), int(main_page_size), physical,
        valid_counts_out is not None)
    return out


def qsa_store_cache_rows(cache: torch.Tensor, slot_mapping: torch.Tensor,
                         rows: torch.Tensor) -> None:
    """Write bf16 raw or compressed key rows into cache pages at their slots
    (ops/qsa.py:691-706)."""
    if rows.ndim == 3:
        rows = rows[:, 0]
    if not rows.shape[0]:
        return
    torch.ops.yulan_qsa_kernels.store_cache_rows(cache, slot_mapping, rows)


def qsa_compress_groups_with_ratio(
    raw_keys: torch.Tensor,
    raw_positions: torch.Tensor,
    compressor_state_cache: torch.Tensor,
    compressor_state_block_table: torch.Tensor,
    token_to_req: torch.Tensor,
    query_start_loc: torch.Tensor,
    logical_positions: torch.Tensor,
    compressed_slots: torch.Tensor,
    compress_ratio: int,
    rope_cache: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 mean of each complete group across the prior ring and the current
    chunk, and the group's first position (ops/qsa.py:709-750). Returns
    ``(pooled [rows, 1, dim], first_positions [rows, 3] int64)``."""
    rows = token_to_req.numel()
    pooled = torch.empty((rows, 1, raw_keys.shape[2]), dtype=raw_keys.dtype,
                         device=raw_keys.device)
    first_positions = torch.empty((rows, 3), dtype=torch.int64, device=raw_keys.device)
    if not rows:
        return pooled, first_positions
    torch.ops.yulan_qsa_kernels.compress_groups(
        raw_keys, raw_positions if rope_cache is not None else None, compressor_state_cache,
        rope_cache, compressor_state_block_table, token_to_req, query_start_loc,
        logical_positions, compressed_slots, int(compress_ratio), pooled, first_positions)
    return pooled, first_positions
