"""Known-answer vectors (tests/golden/qsa_golden.json, written by
tests/golden/make_golden.py from the pure-Python statements in restate.py):
the oracle on the CPU and the HIP kernels on the GPU must reproduce them."""

import json
from pathlib import Path

import pytest
import torch

import oracle

GOLDEN = json.loads((Path(__file__).parent / "golden" / "qsa_golden.json").read_text())
DEV = "cuda:0"


def _scores(bits):
    return torch.tensor([b - (1 << 32) if b >= 1 << 31 else b for b in bits],
                        dtype=torch.int32).view(torch.float32)


def _expand_inputs(case):
    rows = case["rows"]
    width = max(len(r["bits"]) for r in rows)
    scores = torch.zeros(len(rows), width)
    for i, r in enumerate(rows):
        scores[i, :len(r["bits"])] = _scores(r["bits"])
    lengths = torch.tensor([r["length"] for r in rows], dtype=torch.int32)
    positions = torch.tensor([r["position"] for r in rows], dtype=torch.int64)
    t2r = torch.tensor([r["request"] for r in rows], dtype=torch.int32)
    seq = torch.tensor(case["seq_lens"], dtype=torch.int32)
    table = torch.tensor(case["table"], dtype=torch.int32)
    want = torch.tensor([r["out"] for r in rows], dtype=torch.int32)
    counts = torch.tensor([r["count"] for r in rows], dtype=torch.int32)
    return scores, lengths, positions, t2r, seq, table, want, counts


def _indexer_inputs():
    g = GOLDEN["indexer"]
    q = torch.tensor(g["q"], dtype=torch.float32).to(torch.bfloat16)
    cache = torch.tensor(g["cache"], dtype=torch.float32).to(torch.bfloat16).unsqueeze(2)
    table = torch.tensor(g["table"], dtype=torch.int32)
    vis = torch.tensor(g["visible"], dtype=torch.int32)
    return g, q, cache, table, vis


def _attention_inputs():
    g = GOLDEN["attention"]
    q = torch.tensor(g["q"], dtype=torch.float32).to(torch.bfloat16)
    k = torch.tensor(g["k"], dtype=torch.float32).to(torch.bfloat16)
    v = torch.tensor(g["v"], dtype=torch.float32).to(torch.bfloat16)
    idx = torch.tensor(g["indices"], dtype=torch.int32)
    counts = torch.tensor(g["counts"], dtype=torch.int32)
    want = torch.tensor(g["out"], dtype=torch.float64)
    return q, k, v, idx, counts, want


# --------------------------------------------------------------------------- oracle (CPU)

@pytest.mark.parametrize("case", range(len(GOLDEN["topk"])))
def test_oracle_topk_golden(case):
    c = GOLDEN["topk"][case]
    got = oracle.topk_ids(_scores(c["bits"])[None], torch.tensor([c["length"]], dtype=torch.int32),
                          c["k"])
    assert got[0].tolist() == c["ids"]


@pytest.mark.parametrize("case", range(len(GOLDEN["topk_expand"])))
def test_oracle_topk_expand_golden(case):
    c = GOLDEN["topk_expand"][case]
    scores, lengths, positions, t2r, seq, table, want, counts = _expand_inputs(c)
    got, got_counts = oracle.topk_expand(scores, lengths, positions, seq, t2r,
                                         table if c["physical"] else None, c["width"], c["ratio"],
                                         c["page"], c["physical"])
    assert torch.equal(got, want)
    assert torch.equal(got_counts, counts)


def test_oracle_indexer_golden():
    g, q, cache, table, vis = _indexer_inputs()
    cols = len(g["table"][0]) * g["cache_page"]
    got = oracle.indexer_scores_decode(q, cache, table, vis, 1, cols)
    for r, row in enumerate(g["scores"]):
        assert got[r, :len(row)].tolist() == row        # exact: every value is representable


def test_oracle_attention_golden():
    q, k, v, idx, counts, want = _attention_inputs()
    table = torch.zeros(1, 1, dtype=torch.int32)
    t2r = torch.zeros(q.shape[0], dtype=torch.int32)
    got = oracle.sparse_attention(q, k, v, idx, table, t2r, indices_are_physical=True,
                                  valid_counts=counts)
    assert torch.allclose(got.double(), want, atol=1e-5, rtol=0)


# --------------------------------------------------------------------------- kernels (GPU)

@pytest.mark.gpu
def test_kernels_topk_golden():
    for c in GOLDEN["topk"]:
        out = torch.full((1, c["k"]), -5, dtype=torch.int32, device=DEV)
        torch.ops.yulan_qsa_kernels.topk(_scores(c["bits"])[None].to(DEV),
                                         torch.tensor([c["length"]], dtype=torch.int32, device=DEV),
                                         out)
        assert out[0].tolist() == c["ids"]


@pytest.mark.gpu
def test_kernels_topk_expand_golden():
    from qsa_vllm_amd.ops import topk_expand
    for c in GOLDEN["topk_expand"]:
        scores, lengths, positions, t2r, seq, table, want, counts = _expand_inputs(c)
        out = torch.full_like(want, -5).to(DEV)
        got_counts = torch.full_like(counts, -5).to(DEV)
        topk_expand(scores.to(DEV), lengths.to(DEV), positions.to(DEV), seq.to(DEV), t2r.to(DEV),
                    out, c["ratio"], main_block_table=table.to(DEV) if c["physical"] else None,
                    main_page_size=c["page"], valid_counts_out=got_counts)
        assert torch.equal(out.cpu(), want), (c["ratio"], c["page"], c["physical"])
        assert torch.equal(got_counts.cpu(), counts)


@pytest.mark.gpu
def test_kernels_indexer_golden():
    g, q, cache, table, vis = _indexer_inputs()
    cols = len(g["table"][0]) * g["cache_page"]
    logits = torch.full((2, cols), float("nan"), device=DEV)
    torch.ops.yulan_qsa_kernels.indexer_decode(q.to(DEV), cache.to(DEV), table.to(DEV),
                                               vis.to(DEV), logits, 1)
    got = logits.cpu()
    for r, row in enumerate(g["scores"]):
        assert got[r, :len(row)].tolist() == row


@pytest.mark.gpu
def test_kernels_attention_golden():
    from qsa_vllm_amd.ops import qsa_sparse_paged_attention
    q, k, v, idx, counts, want = _attention_inputs()
    table = torch.zeros(1, 1, dtype=torch.int32, device=DEV)
    t2r = torch.zeros(q.shape[0], dtype=torch.int32, device=DEV)
    for splits in (1, 2):
        out = qsa_sparse_paged_attention(q.to(DEV), k.to(DEV), v.to(DEV), idx.to(DEV), table, t2r,
                                         use_decode_kernel=True, indices_are_physical=True,
                                         valid_counts=counts.to(DEV), decode_config=(32, splits, 4))
        err = (out.cpu().double() - want).abs()
        assert err.max() <= 2e-2 and err.mean() <= 2e-3, splits


# --------------------------------------------------------------------------- preparation

def _bf(rows):
    return torch.tensor(rows, dtype=torch.float32).to(torch.bfloat16)


def _prepare_inputs(device="cpu"):
    from types import SimpleNamespace
    g = GOLDEN["prepare"]
    heads, dim, mdim = g["heads"], g["dim"], g["main_dim"]
    tokens = len(g["positions"])
    i64 = lambda v: torch.tensor(v, dtype=torch.int64, device=device)  # noqa: E731
    i32 = lambda v: torch.tensor(v, dtype=torch.int32, device=device)  # noqa: E731
    main = _bf(g["main_cache"]).view(len(g["main_cache"]), g["main_page"], 1, 2 * mdim).to(device)
    raw = SimpleNamespace(slot_mapping=i64(g["state_slots"]), block_table=i32(g["state_table"]),
                          query_start_loc=i32(g["query_start_loc"]),
                          logical_positions=i64(g["positions"]))
    comp = SimpleNamespace(slot_mapping=i64(g["comp_slots"]), k_work_metadata=i32(g["k_work"]))
    args = (_bf(g["index_qk"]).to(device), i64(g["positions"]), _bf(g["q_gamma"]).to(device),
            _bf(g["k_gamma"]).to(device), _bf(g["table"]).to(device), g["eps"], raw, comp,
            _bf(g["state_cache"]).to(device), _bf(g["comp_cache"]).to(device),
            _bf(g["main_key"]).view(tokens, 1, mdim).to(device),
            _bf(g["main_value"]).view(tokens, 1, mdim).to(device),
            main[..., :mdim], main[..., mdim:], i64(g["main_slots"]))
    kwargs = dict(num_index_heads=heads, index_head_dim=dim, rotary_dim=g["rotary"],
                  compress_ratio=g["ratio"])
    return g, args, kwargs, main


def _check_prepare(g, query, args, main):
    assert query.float().cpu().tolist() == g["query"]
    assert args[8].float().cpu().tolist() == g["state_after"]
    assert args[9].float().cpu().tolist() == g["comp_after"]
    assert main.float().cpu().view(len(g["main_after"]), g["main_page"], -1).tolist() == g["main_after"]


def test_oracle_norm_rope_golden():
    g = GOLDEN["norm_rope"]
    got = oracle.norm_rope(_bf(g["x"]), torch.tensor(g["positions"]), _bf(g["gamma"]),
                           _bf(g["table"]), g["eps"], g["rotary"])
    assert got.float().tolist() == g["out"]


def test_oracle_prepare_golden():
    g, args, kwargs, main = _prepare_inputs()
    query = oracle.prepare(*args, **kwargs)
    _check_prepare(g, query, args, main)


@pytest.mark.gpu
def test_kernels_norm_rope_golden():
    from qsa_vllm_amd.ops import IndexerRMSNorm, indexer_norm_rope
    g = GOLDEN["norm_rope"]
    norm = IndexerRMSNorm(g["dim"], g["eps"])
    norm.weight.data = _bf(g["gamma"])
    x = _bf(g["x"]).view(len(g["x"]), 1, g["dim"]).to(DEV)
    got = indexer_norm_rope(x, norm.to(DEV), torch.tensor(g["positions"], device=DEV),
                            _bf(g["table"]).to(DEV), g["rotary"])
    assert got.view(len(g["x"]), g["dim"]).float().cpu().tolist() == g["out"]


@pytest.mark.gpu
def test_kernels_prepare_golden():
    from qsa_vllm_amd.ops import qsa_prepare
    g, args, kwargs, main = _prepare_inputs(DEV)
    query = qsa_prepare(*args, **kwargs)
    torch.cuda.synchronize()
    _check_prepare(g, query, args, main)
