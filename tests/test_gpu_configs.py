"""GPU parity at the benchmark workloads' own full sizes.

Each workload runs through the plugin's entry points exactly as a serving step
does (``select_paged_tokens`` then ``qsa_sparse_paged_attention``), then:

* top-k / expansion / counts are bit-exact against ``oracle.topk_expand`` on
  the indexer kernel's own fp32 logits (every row in decode; every request's
  first and last rows, every logits-span boundary and 2048 random rows in
  prefill);
* indexer logits are within fp32 accumulation error of the oracle's scores;
* attention is within max-abs 2e-2 / mean-abs 2e-3 of the oracle's fp32 math
  over the same selection (every decode row; 256 sampled prefill rows);
* invariants that hold for every row are checked on every row (valid prefix of
  the closed-form count, ascending page-aligned blocks, causal tail, -1 padding).
"""

import pytest
import torch

import oracle
from qsa_vllm_amd import _lib
from qsa_vllm_amd.graph_dispatch import decode_logits_columns, prefill_logits_width
from qsa_vllm_amd.ops import qsa_sparse_paged_attention, select_paged_tokens
from qsa_vllm_amd.ops.indexer import _LOGITS_CAP_BYTES
from qsa_vllm_amd.workloads import make_workload
from tests.selection_checks import closed_form_counts, logical_invariants

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def _note(msg):
    print(f"[case] {msg}", flush=True)


def _attn_check(got, want, what):
    err = (got.float().cpu() - want).abs()
    _note(f"{what}: max_abs={err.max().item():.3e} mean_abs={err.mean().item():.3e}")
    assert err.max().item() <= MAX_ABS and err.mean().item() <= MEAN_ABS, what


def _score_check(got_row, q_row, keys, want_row, what):
    """fp32 accumulation bound: |err| <= 2e-5 * sum_h |q_h| . |k| * D^-0.5 + 1e-6."""
    dim = q_row.shape[-1]
    tol = 2e-5 * (q_row.float().abs() @ keys.float().abs().T).sum(0) * dim ** -0.5 + 1e-6
    assert ((got_row - want_row).abs() <= tol).all(), what


def _keys(index_cache, index_table, req, n):
    c = torch.arange(n)
    page = index_cache.shape[1]
    return index_cache[index_table[req, c // page].long(), c % page, 0]


def _decode_case(name, **overrides):
    wl = make_workload(name, device=DEV, **overrides)
    s = wl.shape
    rows = wl.rows
    idx = torch.full((rows, s.width), -9, dtype=torch.int32, device=DEV)
    counts = torch.full((rows,), -9, dtype=torch.int32, device=DEV)
    select_paged_tokens(wl.q_index, wl.index_cache, wl.index_table, wl.token_to_req, wl.positions,
                        wl.seq_lens, s.token_topk, s.compress_ratio, idx,
                        query_start_loc=wl.query_start_loc, max_query_len=1,
                        max_seq_len=wl.max_seq_len, num_decodes=rows, num_decode_tokens=rows,
                        visible_blocks=wl.visible, main_block_table=wl.block_table,
                        main_page_size=s.page_size, valid_counts_out=counts)
    out = torch.full_like(wl.q, float("nan"))
    qsa_sparse_paged_attention(wl.q, wl.k_cache, wl.v_cache, idx, wl.block_table,
                               wl.token_to_req, out, use_decode_kernel=True,
                               indices_are_physical=True, valid_counts=counts)
    # The logits the selection used: same kernel, same width class.
    cols = decode_logits_columns(wl.max_seq_len, s.compress_ratio,
                                 wl.index_table.shape[1] * wl.index_cache.shape[1])
    logits = torch.full((rows, cols), float("nan"), device=DEV)
    torch.ops.yulan_qsa_kernels.indexer_decode(wl.q_index, wl.index_cache, wl.index_table,
                                               wl.visible, logits, 1)
    torch.cuda.synchronize()
    return wl, idx.cpu(), counts.cpu(), out, logits.cpu(), cols


def _check_decode(wl, idx, counts, out, logits, cols, score_rows):
    s = wl.shape
    rows = wl.rows
    cpu = {n: getattr(wl, n).cpu() for n in ("visible", "positions", "seq_lens", "token_to_req",
                                             "block_table", "q_index", "index_table", "q")}
    # counts: closed form
    want_counts = closed_form_counts(cpu["positions"], cpu["seq_lens"], cpu["token_to_req"],
                                      s.compress_ratio, s.token_topk // s.compress_ratio)
    assert torch.equal(counts.long(), want_counts)
    # top-k + expansion: bit-exact on the kernel's logits, every row
    want_idx, want_c = oracle.topk_expand(logits, cpu["visible"], cpu["positions"],
                                          cpu["seq_lens"], cpu["token_to_req"],
                                          cpu["block_table"], s.width, s.compress_ratio,
                                          s.page_size, True)
    assert torch.equal(idx, want_idx), "top-k/expand differs from the oracle"
    assert torch.equal(counts, want_c)
    # indexer scores against the oracle
    index_cache = wl.index_cache.cpu()
    for r in score_rows:
        n = min(int(cpu["visible"][r]), cols)
        keys = _keys(index_cache, cpu["index_table"], r, n)
        want = oracle.indexer_scores_decode(cpu["q_index"][r:r + 1], index_cache,
                                            cpu["index_table"][r:r + 1], cpu["visible"][r:r + 1],
                                            1, cols)[0]
        _score_check(logits[r, :n], cpu["q_index"][r], keys, want[:n], f"scores row {r}")
        assert torch.isnan(logits[r, n:]).all(), "columns beyond visible stay untouched"
    # attention: every row
    kv = wl.kv_cache.cpu()
    d = s.head_dim
    want = oracle.sparse_attention(cpu["q"], kv[..., :d], kv[..., d:], want_idx,
                                   cpu["block_table"], cpu["token_to_req"],
                                   indices_are_physical=True, valid_counts=want_c)
    _attn_check(out, want, f"{s.name} attention, all {rows} rows")


def test_decode_32k_full_size():
    """decode batch 64, context U[8192, 32768], 16q/2kv x 128, top-k 2048 tokens."""
    _note("decode_32k full size")
    wl, idx, counts, out, logits, cols = _decode_case("decode_32k")
    _check_decode(wl, idx, counts, out, logits, cols, score_rows=range(0, wl.rows, 4))


def test_decode_32k_serving_width():
    """decode_32k with page tables sized for max-model-len 524288: the decode
    logits take the 32768-column width class. The selection and the output are
    those of the tight-table workload (same data, same rows)."""
    _note("decode_32k at the 32768-column width class")
    wl, idx, counts, out, logits, cols = _decode_case("decode_32k_serving_width")
    assert cols == 32768 and wl.index_table.shape[1] * wl.index_cache.shape[1] == 32768
    _check_decode(wl, idx, counts, out, logits, cols, score_rows=range(0, wl.rows, 8))
    tight = _decode_case("decode_32k")
    assert torch.equal(idx, tight[1]) and torch.equal(counts, tight[2])
    assert torch.equal(out, tight[3]), "output must not depend on the width class"


def test_decode_long_skew_full_size():
    """decode batch 8, context lognormal (median 64k) in [16k, 128k]: rows of up
    to 8192 compressed keys, split-K attention over few rows."""
    _note("decode_long_skew full size")
    wl, idx, counts, out, logits, cols = _decode_case("decode_long_skew")
    assert int(wl.visible.max()) > 4096, "the workload should hold long rows"
    _check_decode(wl, idx, counts, out, logits, cols, score_rows=range(wl.rows))


def test_prefill_8k_on_16k_full_size():
    """4 requests x 8192 new tokens on a 16384-token prefix (32768 logical rows),
    through select_paged_tokens' logits spans, then logical sparse attention."""
    _note("prefill_8k_on_16k full size")
    wl = make_workload("prefill_8k_on_16k", device=DEV)
    s = wl.shape
    rows = wl.rows
    k = s.token_topk // s.compress_ratio
    idx = torch.full((rows, s.width), -9, dtype=torch.int32, device=DEV)
    select_paged_tokens(wl.q_index, wl.index_cache, wl.index_table, wl.token_to_req, wl.positions,
                        wl.seq_lens, s.token_topk, s.compress_ratio, idx,
                        query_start_loc=wl.query_start_loc, max_query_len=wl.max_query_len,
                        max_seq_len=wl.max_seq_len, visible_blocks=wl.visible)
    out = torch.full_like(wl.q, float("nan"))
    qsa_sparse_paged_attention(wl.q, wl.k_cache, wl.v_cache, idx, wl.block_table,
                               wl.token_to_req, out)
    width = prefill_logits_width(wl.max_seq_len, s.compress_ratio,
                                 wl.index_table.shape[1] * wl.index_cache.shape[1])
    span = max(1, int(_lib.load().qsa_indexer_prefill_span_rows(width, _LOGITS_CAP_BYTES)))
    assert rows > span, "the workload should take several logits spans"
    # One launch over every row (a different launch shape from the spans: the
    # logits must not depend on it).
    logits = torch.full((rows, width), float("nan"), device=DEV)
    torch.ops.yulan_qsa_kernels.indexer_prefill(wl.q_index, wl.index_cache, wl.index_table,
                                                wl.query_start_loc, wl.visible, logits, 0, rows,
                                                wl.max_query_len)
    torch.cuda.synchronize()
    _note(f"rows={rows} width={width} span={span}")

    # invariants on every row, on the device
    logical_invariants(idx, wl.positions, wl.seq_lens, wl.token_to_req, wl.visible,
                        s.compress_ratio, k)
    assert torch.isfinite(out.float()).all()

    # sampled rows: request ends, span boundaries, random rows
    qsl = wl.query_start_loc.cpu().tolist()
    sample = set()
    for a, b in zip(qsl[:-1], qsl[1:]):
        sample.update((a, a + 1, b - 2, b - 1))
    for a in range(span, rows, span):
        sample.update((a - 1, a))
    g = torch.Generator().manual_seed(33)
    sample.update(torch.randperm(rows, generator=g)[:2048].tolist())
    sample = sorted(sample)
    sel = torch.tensor(sample)
    cpu = {n: getattr(wl, n).cpu() for n in ("visible", "positions", "seq_lens", "token_to_req",
                                             "block_table", "q_index", "index_table", "q",
                                             "query_start_loc")}
    got_logits = logits[sel.to(DEV)].cpu()
    want_idx, _ = oracle.topk_expand(got_logits, cpu["visible"][sel], cpu["positions"][sel],
                                     cpu["seq_lens"], cpu["token_to_req"][sel],
                                     torch.zeros(1, 1, dtype=torch.int32), s.width,
                                     s.compress_ratio, s.page_size, False)
    assert torch.equal(idx[sel.to(DEV)].cpu(), want_idx), "top-k/expand differs from the oracle"

    # indexer scores against the oracle on the boundary rows and 32 random ones
    index_cache = wl.index_cache.cpu()
    score_rows = sorted(set(sample[:8] + sample[-8:] + [r for r in sample if r % span in (0, span - 1)]
                            + sample[::max(1, len(sample) // 32)]))
    for r in score_rows:
        req = int(cpu["token_to_req"][r])
        want = oracle.indexer_scores_prefill(cpu["q_index"], index_cache, cpu["index_table"],
                                             cpu["query_start_loc"], cpu["visible"], r, 1,
                                             width)[0]
        n = min(int(cpu["visible"][r]), width)
        assert n > 0
        keys = _keys(index_cache, cpu["index_table"], req, n)
        got = logits[r].cpu()
        _score_check(got[:n], cpu["q_index"][r], keys, want[:n], f"scores row {r}")
        assert torch.isnan(got[n:]).all(), "columns beyond visible stay untouched"

    # attention against the oracle on 256 sampled rows (logical ids through the table)
    att = torch.tensor(sample[::max(1, len(sample) // 256)])
    kv = wl.kv_cache.cpu()
    d = s.head_dim
    want = oracle.sparse_attention(cpu["q"][att], kv[..., :d], kv[..., d:], idx[att.to(DEV)].cpu(),
                                   cpu["block_table"], cpu["token_to_req"][att])
    _attn_check(out[att.to(DEV)], want, f"prefill attention, {len(att)} sampled rows")
