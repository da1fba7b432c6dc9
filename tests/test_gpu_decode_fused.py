"""Decode selection + attention in one op (``decode_select_attend``) against
the two calls it replaces on the same logits: ``topk_expand`` to physical
slots with counts, then the sparse attention over them with ``valid_counts``.
Both paths run the same device code (the top-k's whole-row selection and the
attention's tile loop), so the selection, its counts and the attention output
must agree bit for bit, on the shapes that run as one launch and on those that
fall back to two calls."""

import pytest
import torch

import qsa_vllm_amd.ops  # noqa: F401  (registers torch.ops.yulan_qsa_kernels)
from qsa_vllm_amd import _lib
from qsa_vllm_amd.graph_dispatch import decode_logits_columns
from qsa_vllm_amd.workloads import make_workload

pytestmark = pytest.mark.gpu

# (name, overrides of decode_32k, expected to run as one launch)
CASES = [
    ("decode_32k", {}, True),
    ("decode_32k_gate", {"gate": True, "seed": 11}, True),
    ("short_rows_1024_columns", {"seq_len_min": 16, "seq_len_max": 16384, "seed": 12}, True),
    ("batch_256_two_kv_per_wg", {"batch": 256, "seq_len_min": 2048, "seq_len_max": 16384,
                                 "seed": 13}, True),
    ("dim64_group8", {"num_q_heads": 8, "num_kv_heads": 1, "head_dim": 64, "seed": 14}, True),
    ("dim64_batch256", {"batch": 256, "head_dim": 64, "seq_len_min": 1024,
                        "seq_len_max": 32768, "seed": 15}, True),
    ("batch_16", {"batch": 16, "seed": 16}, True),
    ("batch_1_1024_columns", {"batch": 1, "seq_len_min": 4096, "seq_len_max": 16384,
                              "seed": 19}, True),
    ("batch_8_dim64", {"batch": 8, "head_dim": 64, "gate": True, "seed": 20}, True),
    # Rows of 4096 to 8192 keys (decode_long_skew's lengths) from an
    # 8192-column buffer, selected inside the attention's workgroups.
    ("long_rows_8192_columns", {"batch": 8, "seq_len_min": 65536, "seq_len_max": 131072,
                                "seed": 17}, True),
    # An 8192-column buffer with rows of 32 to 8192 keys: every column's load
    # goes out before the row's length, and rows are selected in the 512 x 4,
    # 512 x 8 and 512 x 16 shapes by length.
    ("mid_class_mixed_rows", {"table_tokens": 131072, "seq_len_min": 512,
                              "seq_len_max": 131072, "seed": 26}, True),
    # Past the widest class the combined kernel takes (32768 columns): two calls.
    ("rows_past_32768_columns", {"batch": 1, "seq_len_min": 655360, "seq_len_max": 655360,
                                 "seed": 25}, False),
    ("head_major_cache", {"kv_layout": "head_major", "seed": 18}, False),
    # The plugin's 32768-column class (max-model-len 524288): rows of at most
    # 2048 keys selected from their first 2048 columns...
    ("serving_width_32768_columns", {"table_tokens": 524288, "seed": 24}, True),
    # ...and rows of 256 to 32768 keys in that class: whole rows of up to 2048
    # and 8192 keys, rows of up to 16384 staged through LDS, longer rows from
    # their two halves, all inside the attention's workgroups.
    # (45 / 10 / 6 / 3 rows, 3.2 M tokens: the K/V views stay under the 4 GB
    # that buffer addressing covers.)
    ("wide_class_long_rows", {"table_tokens": 524288, "seq_len_dist": "lognormal",
                              "lognormal_median": 24576.0, "lognormal_sigma": 1.5,
                              "seq_len_min": 4096, "seq_len_max": 524288, "seed": 38}, True),
]


def _logits(wl):
    s = wl.shape
    cols = decode_logits_columns(wl.max_seq_len, s.compress_ratio,
                                 wl.index_table.shape[1] * wl.index_cache.shape[1])
    logits = torch.empty(wl.rows, cols, dtype=torch.float32, device=wl.device)
    torch.ops.yulan_qsa_kernels.indexer_decode(wl.q_index, wl.index_cache, wl.index_table,
                                               wl.visible, logits, 1)
    return logits


def _requests(wl, pad_row, t2r):
    t2r = wl.token_to_req.clone() if t2r is None else t2r.clone()
    if pad_row:
        t2r[-1] = -1
    return t2r


def _two_calls(wl, logits, num_splits, pad_row, t2r=None):
    s = wl.shape
    idx = torch.full((wl.rows, s.width), -7, dtype=torch.int32, device=wl.device)
    counts = torch.full((wl.rows,), -7, dtype=torch.int32, device=wl.device)
    out = torch.zeros_like(wl.q)
    t2r = _requests(wl, pad_row, t2r)
    torch.ops.yulan_qsa_kernels.topk_expand(logits, wl.visible, wl.positions, wl.seq_lens, t2r,
                                            wl.block_table, idx, counts, s.compress_ratio,
                                            s.page_size, True, True)
    torch.ops.yulan_qsa_kernels.sparse_attention(wl.q, wl.k_cache, wl.v_cache, idx,
                                                 wl.block_table, t2r, out, wl.gate, counts, True,
                                                 num_splits)
    return idx, counts, out


def _one_op(wl, logits, num_splits, pad_row, t2r=None):
    s = wl.shape
    idx = torch.full((wl.rows, s.width), -9, dtype=torch.int32, device=wl.device)
    counts = torch.full((wl.rows,), -9, dtype=torch.int32, device=wl.device)
    out = torch.full_like(wl.q, 3.0)
    t2r = _requests(wl, pad_row, t2r)
    torch.ops.yulan_qsa_kernels.decode_select_attend(
        logits, wl.visible, wl.positions, wl.seq_lens, t2r, wl.block_table, idx, counts,
        s.compress_ratio, wl.q, wl.k_cache, wl.v_cache, out, wl.gate, num_splits)
    return idx, counts, out


def _check(wl, logits, num_splits, pad_row=False, t2r=None):
    want = _two_calls(wl, logits, num_splits, pad_row, t2r)
    got = _one_op(wl, logits, num_splits, pad_row, t2r)
    torch.cuda.synchronize()
    assert torch.equal(got[0], want[0]), "selection differs"
    assert torch.equal(got[1], want[1]), "counts differ"
    assert torch.equal(got[2].view(torch.int16), want[2].view(torch.int16)), "output differs"
    return want


@pytest.mark.parametrize("name,over,fused", CASES, ids=[c[0] for c in CASES])
def test_decode_select_attend_matches_two_calls(name, over, fused):
    print(f"[case] decode_select_attend {name}", flush=True)
    wl = make_workload("decode_32k", device="cuda", **over)
    s = wl.shape
    logits = _logits(wl)
    rule = _lib.load().qsa_decode_select_attention_fuses(
        wl.rows, logits.shape[1], s.width, s.compress_ratio, s.num_q_heads, s.num_kv_heads,
        s.head_dim)
    # The rule assumes buffer-addressable (token-major) caches; head-major ones
    # always run two calls.
    assert bool(rule) == (fused or s.kv_layout != "token_major"), (rule, fused)
    idx, counts, out = _check(wl, logits, 0)
    assert int(counts.min()) >= 0 and bool(out.abs().amax() > 0)


@pytest.mark.parametrize("num_splits", [1, 4])
def test_decode_select_attend_explicit_splits(num_splits):
    print(f"[case] decode_select_attend decode_32k splits {num_splits}", flush=True)
    wl = make_workload("decode_32k", device="cuda", seed=21)
    _check(wl, _logits(wl), num_splits)


def test_decode_select_attend_padding_row():
    """A row with no request (token_to_req -1) selects nothing: count 0, an
    all -1 index row and a zero output row, on both paths."""
    print("[case] decode_select_attend padding row", flush=True)
    wl = make_workload("decode_32k", device="cuda", seed=22)
    idx, counts, out = _check(wl, _logits(wl), 0, pad_row=True)
    assert int(counts[-1]) == 0 and bool((idx[-1] == -1).all())
    assert not bool(out[-1].any())


@pytest.mark.parametrize("table_tokens", [None, 131072, 524288],
                         ids=["2048_columns", "8192_columns", "32768_columns"])
@pytest.mark.parametrize("mapping", ["reversed", "pairs"])
def test_decode_select_attend_request_mapping(mapping, table_tokens):
    """Rows whose request is not their own index: the combined kernel loads
    the page-table entries of row r's table row ahead of the request and must
    load them again from the right row. Reversed requests, and two rows per
    request (token_to_req[r] = r // 2), against the two calls, in each of the
    combined kernel's buffer classes (2048, 8192 and 32768 columns; the
    8192-column one with rows of 512 to 8192 keys)."""
    print(f"[case] decode_select_attend request mapping {mapping} {table_tokens}", flush=True)
    over = {} if table_tokens is None else {"table_tokens": table_tokens}
    if table_tokens == 131072:
        over.update(seq_len_min=8192, seq_len_max=131072)
    wl = make_workload("decode_32k", device="cuda", seed=23, **over)
    rows = wl.rows
    r = torch.arange(rows, dtype=torch.int32, device=wl.device)
    t2r = (rows - 1 - r) if mapping == "reversed" else r // 2
    idx, counts, out = _check(wl, _logits(wl), 0, t2r=t2r)
    assert int(counts.min()) >= 0 and bool(out.abs().amax() > 0)


def test_decode_select_attend_plugin_entry():
    """ops.decode_select_attend (scoring + the combined op) against the
    plugin's two calls: select_paged_tokens with physical slots, then
    qsa_sparse_paged_attention with valid_counts."""
    from qsa_vllm_amd.ops import decode_select_attend, qsa_sparse_paged_attention, \
        select_paged_tokens

    print("[case] ops.decode_select_attend decode_32k", flush=True)
    wl = make_workload("decode_32k", device="cuda", seed=23, gate=True)
    s = wl.shape
    idx_a = torch.empty(wl.rows, s.width, dtype=torch.int32, device=wl.device)
    cnt_a = torch.empty(wl.rows, dtype=torch.int32, device=wl.device)
    out_a = torch.zeros_like(wl.q)
    select_paged_tokens(wl.q_index, wl.index_cache, wl.index_table, wl.token_to_req,
                        wl.positions, wl.seq_lens, s.token_topk, s.compress_ratio, idx_a,
                        query_start_loc=wl.query_start_loc, max_query_len=1,
                        max_seq_len=wl.max_seq_len, num_decodes=wl.rows,
                        num_decode_tokens=wl.rows, visible_blocks=wl.visible,
                        main_block_table=wl.block_table, main_page_size=s.page_size,
                        valid_counts_out=cnt_a)
    qsa_sparse_paged_attention(wl.q, wl.k_cache, wl.v_cache, idx_a, wl.block_table,
                               wl.token_to_req, out_a, output_gate=wl.gate,
                               use_decode_kernel=True, indices_are_physical=True,
                               valid_counts=cnt_a)
    idx_b = torch.empty_like(idx_a)
    cnt_b = torch.empty_like(cnt_a)
    out_b = torch.zeros_like(wl.q)
    decode_select_attend(wl.q_index, wl.index_cache, wl.index_table, wl.visible, wl.q,
                         wl.k_cache, wl.v_cache, wl.block_table, wl.token_to_req, wl.positions,
                         wl.seq_lens, s.token_topk, s.compress_ratio, wl.max_seq_len, idx_b,
                         cnt_b, out_b, output_gate=wl.gate)
    torch.cuda.synchronize()
    assert torch.equal(idx_a, idx_b) and torch.equal(cnt_a, cnt_b)
    assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16))


def test_decode_select_attend_graph_replays():
    """Captured in a HIP graph and replayed three times over fresh queries
    written between replays: every replay equals the eager two calls."""
    print("[case] decode_select_attend graph replays", flush=True)
    wl = make_workload("decode_32k", device="cuda", seed=24)
    s = wl.shape
    logits = _logits(wl)
    idx = torch.empty(wl.rows, s.width, dtype=torch.int32, device=wl.device)
    counts = torch.empty(wl.rows, dtype=torch.int32, device=wl.device)
    out = torch.zeros_like(wl.q)

    def run():
        torch.ops.yulan_qsa_kernels.decode_select_attend(
            logits, wl.visible, wl.positions, wl.seq_lens, wl.token_to_req, wl.block_table, idx,
            counts, s.compress_ratio, wl.q, wl.k_cache, wl.v_cache, out, None, 0)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    gen = torch.Generator(device=wl.device)
    for rep in range(3):
        gen.manual_seed(100 + rep)
        logits.copy_(torch.randn(logits.shape, generator=gen, device=wl.device))
        wl.q.copy_(torch.randn(wl.q.shape, generator=gen, device=wl.device).to(wl.q.dtype))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = _two_calls(wl, logits, 0, False)
        torch.cuda.synchronize()
        assert torch.equal(idx, want[0]) and torch.equal(counts, want[1]), rep
        assert torch.equal(out.view(torch.int16), want[2].view(torch.int16)), rep
