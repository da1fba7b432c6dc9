"""One QSA layer step on the path, eager or replayed from a HIP graph.

``qsa_layer_step`` is what the plugin's attention layer runs between its
projection and its output projection (``attention.py:191-214`` with the
indexer's ``forward`` at ``:116-142``): prepare (index-q norm + RoPE,
compression groups, ring commit, main K/V writes), select, attend.

``QSALayerStepGraph`` captures that step once for a batch shape and a decode
logits-width class and replays it. Its inputs are fixed buffers: the
projection rows, the attention query, the output and the metadata builder's
buffers, which ``QSAMetadataBuilder.build`` refreshes before each replay. The
graph holds no host values of a batch besides its shape and width class
(``graph_dispatch.py`` of the reference keys its captured graphs the same way).
"""

from __future__ import annotations

import torch

from .backend import run_qsa
from .graph_dispatch import capture_column_scope, check_decode_graph_batch


def qsa_layer_step(indexer, impl, layer, batch, index_qk, main_key, main_value, query, output,
                   gate=None):
    """Prepare, then ``run_qsa``: select into the layer's top-k buffers
    (physical slots and counts in uniform decode, logical ids otherwise) and
    sparse attention into ``output`` (one op for single-token decode). Returns
    ``output``. A step without metadata (``batch`` is None: vLLM's
    memory-profiling forward, ``attention.py:193-198``) zeroes ``output`` and
    writes nothing else."""
    if batch is None:
        output.zero_()
        return output
    n = batch.num_tokens
    key_cache, value_cache = layer.main_kv_views()
    index_query = indexer.prepare(index_qk[:n], batch.positions, batch.raw, batch.compressed,
                                  main_key[:n], main_value[:n], key_cache, value_cache,
                                  batch.main.slot_mapping)
    return run_qsa(layer, impl, index_query, indexer.compressed_key_cache, query, gate, output,
                   batch.main, batch.compressed, indexer.token_topk, indexer.compress_ratio,
                   batch.token_to_req)


class QSALayerStepGraph:
    """``qsa_layer_step`` captured for a uniform decode batch of one size (a
    mixed batch's decode/prefill split and longest query would be baked into
    the launches; the plugin captures full graphs for uniform decode only).
    ``columns`` is the decode logits-width class pinned during capture (0: the
    compressed page table's capacity; ``SHORT_DECODE_COLUMNS``: rows whose
    compressed length fits it). Capture runs the step once (a warm-up), which
    writes the caches like any step."""

    def __init__(self, indexer, impl, layer, batch, index_qk, main_key, main_value, query,
                 output, gate=None, columns: int = 0):
        if batch.main.max_query_len != 1:
            raise ValueError("graphs are captured for uniform decode batches only")
        self.num_tokens = batch.num_tokens
        self.columns = columns
        self.compress_ratio = indexer.compress_ratio
        args = (indexer, impl, layer, batch, index_qk, main_key, main_value, query, output, gate)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with capture_column_scope(columns), torch.cuda.stream(side):
            qsa_layer_step(*args)  # warm-up: allocator pools and kernel loading
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with capture_column_scope(columns), torch.cuda.graph(self.graph):
            qsa_layer_step(*args)

    def replay(self, batch=None):
        """Replay on the current metadata buffers; ``batch`` (from the same
        builder) is checked against the captured size and width class."""
        if batch is not None:
            check_decode_graph_batch(batch, self.num_tokens, self.columns, self.compress_ratio)
        self.graph.replay()
