"""gfx950 HIP operators of the QSA sparse-attention path (reference ``yulan_qsa_vllm/ops``)."""

from .indexer import qsa_select_paged_decode, qsa_select_paged_prefill, select_paged_tokens
from .qsa import qsa_select_paged_tokens, qsa_sparse_paged_attention
from .topk import topk, topk_expand

__all__ = [
    "qsa_select_paged_decode",
    "qsa_select_paged_prefill",
    "qsa_select_paged_tokens",
    "qsa_sparse_paged_attention",
    "select_paged_tokens",
    "topk",
    "topk_expand",
]
