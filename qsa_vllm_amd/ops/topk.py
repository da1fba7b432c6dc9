"""Exact top-k with lowest-id ties, backed by the gfx950 HIP kernels.

Same functions and call pattern as the reference ``yulan_qsa_vllm/ops/topk.py``
(``topk`` :25-26, ``topk_expand`` :29-39): both forward to
``torch.ops.yulan_qsa_kernels`` with the reference schemas. Importing this
module loads ``libqsa_hip.so`` (raising if it is missing) instead of JIT-building
CUDA sources.
"""

from __future__ import annotations

import torch

from .. import _lib
from . import _torch_ops  # noqa: F401  (registers torch.ops.yulan_qsa_kernels)

_lib.load()


def topk(scores, lengths, output):
    torch.ops.yulan_qsa_kernels.topk(scores, lengths, output)


def topk_expand(scores, lengths, query_positions, sequence_lengths, token_to_req,
                output, compress_ratio, *, main_block_table=None, main_page_size=1,
                valid_counts_out=None):
    """Select blocks and write expanded slots, causal tail and counts in place."""
    torch.ops.yulan_qsa_kernels.topk_expand(
        scores, lengths, query_positions, sequence_lengths, token_to_req,
        main_block_table if main_block_table is not None else output,
        output, valid_counts_out if valid_counts_out is not None else output,
        compress_ratio, main_page_size, main_block_table is not None,
        valid_counts_out is not None,
    )
