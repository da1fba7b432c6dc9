"""Host-side glue of the plugin surface that needs no GPU: the memory-profiling
forward without metadata, the decode-graph replay guard, the indexer gamma's
checkpoint loader (CPU)."""

import pytest
import torch

from qsa_vllm_amd import backend
from qsa_vllm_amd.graph_dispatch import SHORT_DECODE_COLUMNS, check_decode_graph_batch
from qsa_vllm_amd.layer_step import qsa_layer_step
from qsa_vllm_amd.metadata import QSAMetadataBuilder
from qsa_vllm_amd.ops.normalization import IndexerRMSNorm


class _Untouchable:
    """Stands in for every layer object a step without metadata must not use."""

    def __getattr__(self, name):
        raise AssertionError(f"a step without metadata used .{name}")


def test_run_qsa_without_metadata_zeroes_output():
    """``attention.py:193-198``: the profile run has no metadata; the output is
    zeroed and nothing else is touched."""
    out = torch.full((3, 4, 8), 7.0, dtype=torch.bfloat16)
    u = _Untouchable()
    got = backend.run_qsa(u, u, u, u, u, u, out, None, None, 2048, 16, u)
    assert got is out and (out == 0).all()


def test_layer_step_without_metadata_zeroes_output():
    out = torch.full((5, 2, 8), -3.0, dtype=torch.bfloat16)
    u = _Untouchable()
    got = qsa_layer_step(u, u, u, None, u, u, u, u, out, u)
    assert got is out and (out == 0).all()


def _decode_batch(seq_len, requests=2, ratio=16):
    b = QSAMetadataBuilder(compress_ratio=ratio, main_page_size=16, comp_page_size=16,
                           ring_size=ratio, max_num_requests=4, max_num_tokens=8,
                           main_table_width=4, comp_table_width=4, device="cpu")
    table = torch.zeros(requests, 4, dtype=torch.int32)
    return b.build([seq_len - 1] * requests, [1] * requests, table, table, [0] * requests)


def test_decode_graph_guard_width_class():
    """A graph captured for the 32768-column class refuses a batch whose
    longest compressed length needs more columns (the other class's graph);
    the capacity class (0) takes any batch of its size."""
    short = _decode_batch(SHORT_DECODE_COLUMNS * 16)
    check_decode_graph_batch(short, 2, SHORT_DECODE_COLUMNS, 16)
    long = _decode_batch(SHORT_DECODE_COLUMNS * 16 + 16)
    with pytest.raises(ValueError, match="width class"):
        check_decode_graph_batch(long, 2, SHORT_DECODE_COLUMNS, 16)
    check_decode_graph_batch(long, 2, 0, 16)
    with pytest.raises(ValueError, match="captured size"):
        check_decode_graph_batch(short, 3, SHORT_DECODE_COLUMNS, 16)


def test_indexer_gamma_weight_loader():
    """``ops/normalization.py:29``: the gamma carries a checkpoint loader."""
    norm = IndexerRMSNorm(16, 1e-6)
    loaded = torch.arange(16, dtype=torch.bfloat16)
    norm.weight.weight_loader(norm.weight, loaded)
    assert torch.equal(norm.weight.data, loaded)
    with pytest.raises(Exception):
        norm.weight.weight_loader(norm.weight, torch.zeros(8, dtype=torch.bfloat16))


def test_gemm_tuning_file_is_well_formed(tmp_path):
    """The recorded library GEMM choices name their software stack (PyTorch
    rejects the file on any other) and one solution per GEMM shape."""
    from qsa_vllm_amd.gemm_tuning import TUNING_FILE, enable_tuned_gemms

    lines = TUNING_FILE.read_text().splitlines()
    validators = {line.split(",")[1]: line.split(",")[2] for line in lines
                  if line.startswith("Validator,")}
    assert {"PT_VERSION", "HIPBLASLT_VERSION", "ROCBLAS_VERSION", "GCN_ARCH_NAME"} <= set(validators)
    assert validators["GCN_ARCH_NAME"].startswith("gfx950")
    records = [line.split(",") for line in lines if not line.startswith("Validator,")]
    assert len(records) >= 10
    assert len({r[1] for r in records}) == len(records)  # one choice per shape
    assert all(r[1].startswith("tn_") and r[2] for r in records)
    assert enable_tuned_gemms(tmp_path / "missing.csv") is False


@pytest.mark.parametrize("width,config,want", [
    (2063, (64, 8, 4), 8),       # cdiv = 33 -> 32, capped by the target 8
    (2063, (32, 64, 1), 64),     # cdiv = 65 -> 64
    (2063, (64, 64, 1), 32),     # the same target with block_n 64 gives half the splits
    (2063, (16, 1000, 4), 128),  # cdiv = 129 -> 128
    (100, (32, 16, 4), 4),       # cdiv = 4
    (1039, (32, 3, 4), 3),       # a target that is not a power of two is kept
    (1, (64, 16, 4), 1),
    (2063, (32, 0, 4), 1),       # never below one split
    (100000, (1, 5000, 4), 1024),  # never above the library's bound
])
def test_decode_config_split_count(width, config, want):
    """``ops/qsa.py:643-645``: num_splits = min(pow2floor(cdiv(W, block_n)),
    target_splits), from the caller's block_n."""
    from qsa_vllm_amd.ops.qsa import choose_num_splits, config_num_splits
    assert config_num_splits(width, config) == want
    q = torch.empty(4, 16, 128, dtype=torch.bfloat16)
    k = torch.empty(8, 16, 2, 128, dtype=torch.bfloat16)
    idx = torch.empty(4, width, dtype=torch.int32)
    assert choose_num_splits(q, k, idx, True, config) == want


def test_decode_config_ignored_for_prefill_rows():
    """The reference reads ``decode_config`` only for the decode kernel
    (``ops/qsa.py:620-622``); prefill rows take the library's choice."""
    from qsa_vllm_amd import _lib
    from qsa_vllm_amd.ops.qsa import choose_num_splits
    q = torch.empty(64, 16, 128, dtype=torch.bfloat16)
    k = torch.empty(8, 16, 2, 128, dtype=torch.bfloat16)
    idx = torch.empty(64, 2063, dtype=torch.int32)
    lib_choice = _lib.load().qsa_sparse_attention_splits(64, 16, 2, 128, 2063, 0)
    assert choose_num_splits(q, k, idx, False, (16, 1000, 4)) == lib_choice
    assert choose_num_splits(q, k, idx, False, None) == lib_choice
    with pytest.raises(ValueError):
        choose_num_splits(q, k, idx, True, (0, 4, 4))


def test_decode_step_bytes_adds_the_three_launches():
    """The bench's whole-step roofline counts the indexer, the top-k (one
    page-table entry per selected block, at most k per row) and the attention."""
    from qsa_vllm_amd.workloads import (QSAShape, attention_bytes, decode_step_bytes,
                                        indexer_bytes, make_workload, topk_bytes)

    shape = QSAShape("tiny_decode", batch=4, num_q_heads=4, num_kv_heads=1, head_dim=64,
                     page_size=16, compress_ratio=16, index_heads=4, index_dim=64,
                     token_topk=256, seq_len_min=40, seq_len_max=600, seed=0)
    wl = make_workload(shape)
    k = shape.token_topk // shape.compress_ratio
    vis = [int(v) for v in wl.visible]
    assert min(vis) < k < max(vis)  # rows on both sides of k
    want_topk = sum(v * 4 + (shape.width + 1) * 4 + 12 + min(v, k) * 4 for v in vis)
    assert topk_bytes(wl) == want_topk
    counts = shape.token_topk + wl.seq_lens % shape.compress_ratio
    assert decode_step_bytes(wl, counts) == (indexer_bytes(wl) + want_topk
                                             + attention_bytes(wl, counts))
