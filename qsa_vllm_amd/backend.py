"""Attention-side glue of the QSA path, without vLLM.

The reference plugin's backend (``yulan_qsa_vllm/backend.py``) and attention
module (``yulan_qsa_vllm/attention.py``) import vLLM, which only provides their
base classes and the forward context. What they compute on the QSA path is
small and is restated here with the same names and argument meaning, so that
the ops in :mod:`qsa_vllm_amd.ops` can be driven exactly as the plugin drives
them:

* :class:`YuLanQSAMetadata` — the main-attention metadata fields
  (``metadata.py:29-34``).
* :func:`main_kv_views` — K and V views of the vLLM-bound main cache
  (``backend.py:148-153``).
* :class:`YuLanQSAImpl` — zero the output, then sparse attention with the
  decode flags taken from ``max_query_len`` (``backend.py:24-68``).
* :class:`QSACompressedMetadata`, :class:`QSARawMetadata`,
  :class:`YuLanQSAIndexer` and :func:`select_for_layer` — the indexer: index
  query/key preparation and cache writes, then the selection call with the
  main block table and counts passed only in uniform decode
  (``attention.py:79-142``, ``:191-214``).
* :func:`run_qsa` — ``_run_qsa`` from the prepared index query on.

The compressed-cache metadata is produced upstream in vLLM's QSA cache
builder, whose source is not part of the plugin; its fields here follow what
the plugin's consumers read.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .ops.indexer import _visible_blocks, decode_select_attend
from .ops.indexer import select_paged_tokens as qsa_select_paged_tokens  # attention.py:21
from .ops.normalization import IndexerRMSNorm, rotary_cache
from .ops.prepare import qsa_prepare
from .ops.qsa import qsa_sparse_paged_attention


@dataclass
class YuLanQSAMetadata:
    """Main-attention metadata (``metadata.py:29-34``)."""

    num_actual_tokens: int
    max_query_len: int
    block_table: torch.Tensor
    slot_mapping: torch.Tensor


@dataclass
class QSACompressedMetadata:
    """Compressed-key metadata fields the indexer reads (``attention.py:128-142``)."""

    block_table: torch.Tensor
    token_to_req: torch.Tensor
    logical_positions: torch.Tensor
    seq_lens: torch.Tensor
    query_start_loc: torch.Tensor
    max_query_len: int
    max_seq_len: int
    num_decodes: int
    num_decode_tokens: int
    decode_query_len: int = 1
    visible_blocks: torch.Tensor | None = None
    slot_mapping: torch.Tensor | None = None      # qsa_prepare: compressed slot per token
    k_work_metadata: torch.Tensor | None = None   # qsa_prepare: (request, group) items


@dataclass
class QSARawMetadata:
    """Raw-key ring metadata ``qsa_prepare`` reads (``ops/prepare.py:208-209``)."""

    slot_mapping: torch.Tensor
    block_table: torch.Tensor
    query_start_loc: torch.Tensor
    logical_positions: torch.Tensor


class YuLanQSAIndexer:
    """The replicated indexer of a QSA layer (``attention.py:79-142``): index-q
    and compressed-key RMSNorm gammas, the rotary table, the raw-key ring and
    the compressed-key cache. ``forward`` prepares (norm + RoPE, compression
    groups, ring commit, main K/V writes) and selects."""

    def __init__(self, num_heads: int, head_dim: int, compress_ratio: int, token_topk: int,
                 rotary_dim: int, rope_theta: float, eps: float, max_position: int,
                 raw_key_cache: torch.Tensor, compressed_key_cache: torch.Tensor):
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.compress_ratio = compress_ratio
        self.token_topk = token_topk
        self.rotary_dim = rotary_dim
        device = compressed_key_cache.device
        self.q_layernorm = IndexerRMSNorm(head_dim, eps).to(device)
        self.k_layernorm = IndexerRMSNorm(head_dim, eps).to(device)
        self.cos_sin_cache = rotary_cache(max_position, rotary_dim, float(rope_theta), device)
        self.raw_key_cache = raw_key_cache
        self.compressed_key_cache = compressed_key_cache

    @property
    def output_width(self):
        return self.token_topk + self.compress_ratio - 1

    def prepare(self, projected, positions, raw_metadata, compressed_metadata, main_key,
                main_value, main_key_cache, main_value_cache, main_slots):
        """The preparation half of ``forward`` (``attention.py:118-126``): returns
        the normed, rotated index query after the cache writes."""
        return qsa_prepare(
            projected, positions, self.q_layernorm.weight, self.k_layernorm.weight,
            self.cos_sin_cache, self.q_layernorm.variance_epsilon, raw_metadata,
            compressed_metadata, self.raw_key_cache, self.compressed_key_cache, main_key,
            main_value, main_key_cache, main_value_cache, main_slots,
            num_index_heads=self.num_heads, index_head_dim=self.head_dim,
            rotary_dim=self.rotary_dim, compress_ratio=self.compress_ratio)

    def forward(self, projected, positions, raw_metadata, compressed_metadata, out,
                main_key, main_value, main_key_cache, main_value_cache, main_slots,
                *, main_block_table=None, valid_counts_out=None):
        query = self.prepare(projected, positions, raw_metadata, compressed_metadata, main_key,
                             main_value, main_key_cache, main_value_cache, main_slots)
        return select_for_layer(query, self.compressed_key_cache, compressed_metadata, out,
                                self.token_topk, self.compress_ratio, main_key_cache,
                                main_block_table=main_block_table,
                                valid_counts_out=valid_counts_out)


def canonicalize_singleton_dim_strides(t: torch.Tensor) -> torch.Tensor:
    """The same view with every size-1 dim given the stride a contiguous tensor
    of the same trailing shape would have (its value is never used to address
    memory, but kernels may check it)."""
    strides = list(t.stride())
    for d in range(t.dim() - 1, -1, -1):
        if t.size(d) == 1:
            strides[d] = strides[d + 1] * t.size(d + 1) if d + 1 < t.dim() else 1
    return t.as_strided(t.shape, strides)


def main_kv_views(kv_cache: torch.Tensor, head_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """K and V views ``[blocks, page, kv_heads, head_size]`` of the main cache.

    vLLM binds the cache as the logical ``[blocks, kv_heads, page, 2 * head_size]``
    view (K|V interleaved per (token, kv head) row), whichever of the BLNHC / BLHNC
    physical layouts backs it (``backend.py:100-102``); ``backend.py:148-153``
    swaps the head and page dims and splits the last one.
    """
    key_cache, value_cache = kv_cache.transpose(1, 2).split(head_size, dim=-1)
    return (canonicalize_singleton_dim_strides(key_cache),
            canonicalize_singleton_dim_strides(value_cache))


class QSALayerState:
    """The per-layer state the plugin's attention module holds for the path:
    the vLLM-bound main cache and the top-k index/count buffers sized for the
    scheduler's token budget (``attention.py:169-182``)."""

    def __init__(self, kv_cache: torch.Tensor, head_size: int, max_num_batched_tokens: int,
                 output_width: int):
        self.kv_cache = kv_cache
        self.head_size = head_size
        dev = kv_cache.device
        self.topk_indices_buffer = torch.empty(max_num_batched_tokens, output_width,
                                               dtype=torch.int32, device=dev)
        self.topk_counts_buffer = torch.empty(max_num_batched_tokens, dtype=torch.int32,
                                              device=dev)

    def main_kv_views(self):
        return main_kv_views(self.kv_cache, self.head_size)


class YuLanQSAImpl:
    """Sparse paged attention against the layer's K/V heads (``backend.py:24-68``)."""

    def __init__(self, num_heads: int, num_kv_heads: int, head_size: int) -> None:
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_size = head_size
        self.scale = head_size ** -0.5

    def forward(self, layer, query: torch.Tensor, attn_metadata: YuLanQSAMetadata,
                output: torch.Tensor, *, token_to_req: torch.Tensor,
                output_gate: torch.Tensor | None = None) -> torch.Tensor:
        num_tokens = attn_metadata.num_actual_tokens
        key_cache, value_cache = layer.main_kv_views()
        decode = attn_metadata.max_query_len == 1
        # The reference zero-fills the whole output first. The attention
        # writes every element of output[:num_tokens] (a row without a valid
        # slot gets zeros), so only the padded rows past it need the fill.
        output[num_tokens:].zero_()
        qsa_sparse_paged_attention(
            query[:num_tokens], key_cache, value_cache,
            layer.topk_indices_buffer[:num_tokens], attn_metadata.block_table,
            token_to_req[:num_tokens], output[:num_tokens],
            output_gate=output_gate[:num_tokens] if output_gate is not None else None,
            use_decode_kernel=decode, indices_are_physical=decode,
            valid_counts=layer.topk_counts_buffer[:num_tokens] if decode else None)
        return output


def select_for_layer(index_query: torch.Tensor, compressed_key_cache: torch.Tensor,
                     compressed: QSACompressedMetadata, out: torch.Tensor, token_topk: int,
                     compress_ratio: int, main_key_cache: torch.Tensor, *,
                     main_block_table: torch.Tensor | None = None,
                     valid_counts_out: torch.Tensor | None = None) -> torch.Tensor:
    """The selection half of ``YuLanQSAIndexer.forward`` (``attention.py:116-142``),
    taking the already prepared index query."""
    return qsa_select_paged_tokens(
        index_query, compressed_key_cache, compressed.block_table, compressed.token_to_req,
        compressed.logical_positions, compressed.seq_lens, token_topk, compress_ratio, out,
        query_start_loc=compressed.query_start_loc, max_query_len=compressed.max_query_len,
        max_seq_len=compressed.max_seq_len, num_decodes=compressed.num_decodes,
        num_decode_tokens=compressed.num_decode_tokens,
        decode_query_len=compressed.decode_query_len,
        visible_blocks=compressed.visible_blocks, main_block_table=main_block_table,
        main_page_size=main_key_cache.shape[1], valid_counts_out=valid_counts_out)


def run_qsa(layer: QSALayerState, impl: YuLanQSAImpl, index_query: torch.Tensor,
            compressed_key_cache: torch.Tensor, query: torch.Tensor,
            gate: torch.Tensor | None, output: torch.Tensor, main: YuLanQSAMetadata,
            compressed: QSACompressedMetadata, token_topk: int, compress_ratio: int,
            token_to_req: torch.Tensor) -> torch.Tensor:
    """``_run_qsa`` (``attention.py:191-214``) from the prepared index query on:
    select into the layer's top-k buffer (physical slots + counts in uniform
    decode, logical token ids otherwise), then attend. Without metadata (vLLM's
    memory-profiling forward, ``attention.py:193-198``) the output is zeroed
    and nothing else runs."""
    if main is None or compressed is None:
        output.zero_()
        return output
    count = main.num_actual_tokens
    is_decode = main.max_query_len == 1
    key_cache, value_cache = layer.main_kv_views()
    if is_decode and compressed.decode_query_len == 1:
        # One token per request: scoring, then the top-k + expansion and the
        # attention as one op (the same selection into the layer's buffers and
        # the same output as the two calls below).
        t2r = compressed.token_to_req[:count]
        pos = compressed.logical_positions[:count]
        visible = compressed.visible_blocks
        visible = (visible[:count] if visible is not None
                   else _visible_blocks(pos, compressed.seq_lens, t2r, compress_ratio))
        output[count:].zero_()
        decode_select_attend(
            index_query[:count], compressed_key_cache, compressed.block_table, visible,
            query[:count], key_cache, value_cache, main.block_table, t2r, pos,
            compressed.seq_lens, token_topk,
            compress_ratio, compressed.max_seq_len, layer.topk_indices_buffer[:count],
            layer.topk_counts_buffer[:count], output[:count],
            output_gate=gate[:count] if gate is not None else None)
        return output
    select_for_layer(
        index_query[:count], compressed_key_cache, compressed,
        layer.topk_indices_buffer[:count], token_topk, compress_ratio, key_cache,
        main_block_table=main.block_table if is_decode else None,
        valid_counts_out=layer.topk_counts_buffer[:count] if is_decode else None)
    return impl.forward(layer, query, main, output, token_to_req=token_to_req,
                        output_gate=gate)
