"""Indexer preparation and main K/V cache writes (the producers of the path).

Mirrors ``qsa_prepare`` (ops/prepare.py:177-225 of the reference plugin):
same arguments, same results, one launch of ``libqsa_hip.so``. The metadata
objects carry the fields the reference kernel reads:

* ``raw_metadata``: ``slot_mapping`` (int64 [tokens], ring slot per token,
  -1 for none), ``block_table`` (int32 [requests, width], column 0 is the
  request's ring block), ``query_start_loc`` (int32 [requests + 1]) and
  ``logical_positions`` (int64 [tokens]);
* ``compressed_metadata``: ``slot_mapping`` (int64 [tokens], the compressed
  slot of the group that ends at each token, -1 elsewhere) and
  ``k_work_metadata`` (int32 [items, 2]: request, group within the request;
  request < 0 pads).
"""

from __future__ import annotations

import torch

from . import _torch_ops  # noqa: F401  (registers torch.ops.yulan_qsa_kernels)

__all__ = ["qsa_prepare"]


def qsa_prepare(
    index_qk: torch.Tensor,
    positions: torch.Tensor,
    q_norm_weight: torch.Tensor,
    k_norm_weight: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    eps: float,
    raw_metadata,
    compressed_metadata,
    state_cache: torch.Tensor,
    compressed_cache: torch.Tensor,
    main_key: torch.Tensor,
    main_value: torch.Tensor,
    main_key_cache: torch.Tensor,
    main_value_cache: torch.Tensor,
    main_slots: torch.Tensor,
    *,
    num_index_heads: int,
    index_head_dim: int,
    rotary_dim: int,
    compress_ratio: int,
) -> torch.Tensor:
    """RMSNorm + RoPE of the index queries (returned, [tokens, heads, dim] bf16),
    one normalised mean-pooled key per completed compression group into
    ``compressed_cache``, the chunk's last raw keys into the request's ring in
    ``state_cache``, and the main K/V rows into their cache slots
    (ops/prepare.py:49-174)."""
    tokens = index_qk.shape[0]
    query = index_qk.new_empty(tokens, num_index_heads, index_head_dim)
    torch.ops.yulan_qsa_kernels.indexer_prepare(
        index_qk, positions, q_norm_weight, k_norm_weight, cos_sin_cache, float(eps), query,
        state_cache, raw_metadata.slot_mapping, raw_metadata.block_table,
        raw_metadata.query_start_loc, raw_metadata.logical_positions,
        compressed_cache, compressed_metadata.slot_mapping, compressed_metadata.k_work_metadata,
        main_key, main_value, main_key_cache, main_value_cache, main_slots,
        int(num_index_heads), int(index_head_dim), int(rotary_dim), int(compress_ratio))
    return query
