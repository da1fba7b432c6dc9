"""gfx950 HIP operators of the QSA sparse-attention path (reference ``yulan_qsa_vllm/ops``)."""

from .indexer import (decode_select_attend, qsa_select_paged_decode, qsa_select_paged_prefill,
                      select_paged_tokens)
from .normalization import IndexerRMSNorm, indexer_norm_rope, rotary_cache
from .prepare import qsa_prepare
from .qsa import (expand_qsa_block_indices_cuda, qsa_compress_groups_with_ratio,
                  qsa_select_paged_tokens, qsa_sparse_paged_attention, qsa_store_cache_rows)
from .topk import topk, topk_expand

__all__ = [
    "IndexerRMSNorm",
    "decode_select_attend",
    "expand_qsa_block_indices_cuda",
    "qsa_compress_groups_with_ratio",
    "qsa_store_cache_rows",
    "indexer_norm_rope",
    "qsa_prepare",
    "qsa_select_paged_decode",
    "qsa_select_paged_prefill",
    "qsa_select_paged_tokens",
    "qsa_sparse_paged_attention",
    "rotary_cache",
    "select_paged_tokens",
    "topk",
    "topk_expand",
]
