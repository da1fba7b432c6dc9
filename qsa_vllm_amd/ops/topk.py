"""Exact per-row top-k and its expansion to token slots, on the gfx950 kernels.

Entry points of the reference ``yulan_qsa_vllm/ops/topk.py`` (``topk`` :25-26,
``topk_expand`` :29-39) with the same arguments, both running the
``torch.ops.yulan_qsa_kernels`` ops of the reference schemas. Importing this
module loads ``libqsa_hip.so`` and raises if it is missing; nothing is built
at import time.
"""

from __future__ import annotations

import torch

from .. import _lib
from . import _torch_ops  # noqa: F401  (registers torch.ops.yulan_qsa_kernels)

_lib.load()


def topk(scores, lengths, output):
    """Row r of ``output`` ([rows, k] int32) receives the ids of the k largest
    of ``scores[r, :lengths[r]]`` in ascending id order, the lower id winning
    among equal fp32 bit patterns; rows shorter than k get ``0..len-1`` then -1."""
    torch.ops.yulan_qsa_kernels.topk(scores, lengths, output)


def topk_expand(scores, lengths, query_positions, sequence_lengths, token_to_req,
                output, compress_ratio, *, main_block_table=None, main_page_size=1,
                valid_counts_out=None):
    """Top ``output.size(1) // compress_ratio`` blocks per row, written as the
    tokens of each block plus the row's causal tail; logical token ids, or
    physical cache slots through ``main_block_table``; optionally the valid
    count per row.

    The op takes every tensor positionally: when the table or the counts are
    absent, ``output`` stands in for them and the op's ``physical`` /
    ``store_counts`` flags say that they are not to be used.
    """
    physical = main_block_table is not None
    store_counts = valid_counts_out is not None
    torch.ops.yulan_qsa_kernels.topk_expand(
        scores, lengths, query_positions, sequence_lengths, token_to_req,
        main_block_table if physical else output, output,
        valid_counts_out if store_counts else output,
        compress_ratio, main_page_size, physical, store_counts)
