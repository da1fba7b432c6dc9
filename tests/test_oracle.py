"""Pins the CPU oracle against brute force, closed forms and invariants (CPU only)."""

import math
import random

import pytest
import torch

import oracle
from tests import restate


def _f32(values):
    return torch.tensor(values, dtype=torch.float32)


def _bits(values):
    return torch.tensor(values, dtype=torch.int64).to(torch.int32).view(torch.float32)


# --------------------------------------------------------------------------- visible


def test_visible_blocks_closed_form():
    pos = torch.tensor([0, 14, 15, 16, 31, 100, 5, 100], dtype=torch.int64)
    seq = torch.tensor([64, 20], dtype=torch.int32)
    t2r = torch.tensor([0, 0, 0, 0, 1, 1, -1, -1], dtype=torch.int32)
    got = oracle.visible_blocks(pos, seq, t2r, 16).tolist()
    # min((pos+1)//16, seq[req]//16), 0 for padding rows
    assert got == [0, 0, 1, 1, 1, 1, 0, 0]


def test_logits_width_rules():
    assert oracle.decode_logits_columns(32768 * 16, 16, 1 << 20) == 32768
    assert oracle.decode_logits_columns(32768 * 16 + 16, 16, 1 << 20) == 1 << 20
    assert oracle.decode_logits_columns(1000, 16, 2048) == 2048
    assert oracle.prefill_logits_width(24576, 16, 1536) == 1536
    assert oracle.prefill_logits_width(100, 16, 4096) == 64
    assert oracle.prefill_logits_width(0, 16, 4096) == 64       # never below 64 columns
    assert oracle.prefill_logits_width(1100, 16, 4096) == 128
    assert oracle.prefill_logits_width(1025 * 16, 16, 4096) == 1088   # 1025 keys -> 17 x 64


# --------------------------------------------------------------------------- top-k


@pytest.mark.parametrize("scores,k,expected", [
    ([1.0, 3.0, 3.0, 2.0, 3.0], 2, [1, 2]),             # ties -> lowest ids
    ([1.0, 3.0, 3.0, 2.0, 3.0], 4, [1, 2, 3, 4]),
    ([5.0, -0.0, 1.0], 1, [1]),                          # -0.0 is 0x80000000: above all positives
    ([-1.0, 2.0, 7.0], 1, [0]),                          # negatives rank above positives
    ([-1.0, -2.0, 0.5], 1, [1]),                         # larger negative magnitude ranks higher
    ([float("inf"), 1e30, 0.0], 2, [0, 1]),
    ([0.0, 0.0, 0.0, 0.0], 2, [0, 1]),                   # all equal
    ([2.0, 1.0], 5, [0, 1, -1, -1, -1]),                 # length <= k
])
def test_topk_known_answers(scores, k, expected):
    s = _f32(scores)[None]
    got = oracle.topk_ids(s, torch.tensor([len(scores)], dtype=torch.int32), k)
    assert got[0].tolist() == expected


def test_topk_nan_bit_patterns():
    # Positive quiet NaN 0x7fc00000 > +inf 0x7f800000; negative NaN 0xffc00000 is the largest key.
    s = _bits([0x3F800000, 0x7FC00000, 0x7F800000, 0xFFC00000 - (1 << 32), 0x00000001])[None]
    got = oracle.topk_ids(s, torch.tensor([5], dtype=torch.int32), 2)
    assert got[0].tolist() == [1, 3]


def test_topk_matches_rank_counting():
    rng = random.Random(7)
    for trial in range(60):
        n = rng.randint(1, 90)
        k = rng.randint(1, 40)
        pool = [rng.choice([0.0, -0.0, 1.0, 2.5, -3.0, 1e-39, float("inf")])
                if rng.random() < 0.3 else rng.uniform(-4, 4) for _ in range(n)]
        if trial % 3 == 0:  # heavy ties
            pool = [float(rng.randint(0, 3)) for _ in range(n)]
        scores = _f32(pool)
        length = rng.randint(0, n)
        got = oracle.topk_ids(scores[None], torch.tensor([length], dtype=torch.int32), k)[0].tolist()
        want = restate.topk_by_rank(restate.u32_keys(scores), length, k)
        if length > k:
            assert got == want
        else:
            assert got == [i if i < length else -1 for i in range(k)]


# --------------------------------------------------------------------------- expansion


def _random_expand_case(rng, physical):
    ratio = rng.choice([1, 2, 4, 16])
    page = ratio * rng.choice([1, 2]) if rng.random() < 0.7 else rng.choice([3, 5, 272])
    k = rng.randint(1, 6)
    width = k * ratio + ratio - 1
    reqs = rng.randint(1, 3)
    seq_lens = [rng.randint(0, 90) for _ in range(reqs)]
    table_width = max(1, (max(seq_lens) + page - 1) // page + rng.randint(-1, 1))
    table = [[rng.choice([-1] + list(range(50))) if rng.random() < 0.2 else rng.randint(0, 40)
              for _ in range(table_width)] for _ in range(reqs)]
    rows = rng.randint(1, 6)
    t2r = [rng.randint(-1, reqs) for _ in range(rows)]
    pos = []
    for r in t2r:
        sl = seq_lens[r] if 0 <= r < reqs else 10
        pos.append(rng.randint(0, max(0, sl + 3)))
    cols = rng.randint(1, 30)
    lengths = [min(cols, max(0, rng.randint(0, 30))) for _ in range(rows)]
    scores = torch.randn(rows, cols)
    if rng.random() < 0.3:
        scores = scores.round()
    return dict(ratio=ratio, page=page, k=k, width=width, seq_lens=seq_lens, table=table,
                t2r=t2r, pos=pos, lengths=lengths, scores=scores, physical=physical)


@pytest.mark.parametrize("physical", [False, True])
def test_topk_expand_matches_columnwise_statement(physical):
    rng = random.Random(11 + physical)
    for _ in range(150):
        c = _random_expand_case(rng, physical)
        out, counts = oracle.topk_expand(
            c["scores"], torch.tensor(c["lengths"], dtype=torch.int32),
            torch.tensor(c["pos"], dtype=torch.int64), torch.tensor(c["seq_lens"], dtype=torch.int32),
            torch.tensor(c["t2r"], dtype=torch.int32), torch.tensor(c["table"], dtype=torch.int32),
            c["width"], c["ratio"], c["page"], physical)
        blocks = oracle.topk_ids(c["scores"], torch.tensor(c["lengths"], dtype=torch.int32), c["k"])
        for r in range(len(c["t2r"])):
            want, want_count = restate.expand_columns(
                blocks[r].tolist(), c["pos"][r], c["t2r"][r], c["seq_lens"], c["ratio"],
                c["width"], physical, c["table"], c["page"])
            assert out[r].tolist() == want
            assert int(counts[r]) == want_count


def test_topk_expand_hand_built_physical():
    # ratio 4, page 8: blocks 0,1 share logical page 0 -> physical page 5; block 2,3 -> page 2.
    scores = _f32([[1.0, 9.0, 3.0, 8.0, 0.5, 0.1]])
    out, counts = oracle.topk_expand(
        scores, torch.tensor([4], dtype=torch.int32), torch.tensor([17], dtype=torch.int64),
        torch.tensor([18], dtype=torch.int32), torch.tensor([0], dtype=torch.int32),
        torch.tensor([[5, 2, 7]], dtype=torch.int32), 2 * 4 + 3, 4, 8, True)
    # top-2 of visible 4 blocks -> blocks 1 (9.0) and 3 (8.0), ascending; tail = tokens 16, 17.
    # block 1: tokens 4..7 -> page 5 slots 44..47; block 3: tokens 12..15 -> page 2 slots 20..23;
    # tail tokens 16, 17 -> logical page 2 -> physical 7 -> slots 56, 57.
    assert out[0].tolist() == [44, 45, 46, 47, 20, 21, 22, 23, 56, 57, -1]
    assert int(counts[0]) == 10


def test_topk_expand_invariants_logical():
    g = torch.Generator().manual_seed(3)
    rows, r, k = 40, 4, 8
    seq = torch.randint(1, 200, (5,), generator=g, dtype=torch.int32)
    t2r = torch.randint(0, 5, (rows,), generator=g, dtype=torch.int32)
    pos = (torch.rand(rows, generator=g) * seq[t2r.long()].float()).long()
    vis = oracle.visible_blocks(pos, seq, t2r, r)
    scores = torch.randn(rows, 64, generator=g)
    out, counts = oracle.topk_expand(scores, vis, pos, seq, t2r, torch.zeros(1, 1, dtype=torch.int32),
                                     k * r + r - 1, r, 1, False)
    for i in range(rows):
        row = out[i].tolist()
        n = int(counts[i])
        valid = [t for t in row if t >= 0]
        assert row[:len(valid)] == valid                      # valid entries form a prefix
        assert len(valid) == n                                # ... of length count
        assert len(set(valid)) == len(valid)                  # no duplicate tokens
        assert all(t <= int(pos[i]) for t in valid)           # causal
        tail = (int(pos[i]) + 1) % r
        assert valid[-tail:] == list(range(int(pos[i]) + 1 - tail, int(pos[i]) + 1)) if tail else True


# --------------------------------------------------------------------------- indexer


@pytest.mark.parametrize("dql", [1, 2])
def test_indexer_scores_bruteforce(dql):
    """Row r scores request r // dql's keys (``ops/indexer.py:241-279``)."""
    g = torch.Generator().manual_seed(5)
    rows, heads, dim, page, blocks = 3 * dql, 3, 8, 4, 6
    q = (torch.randn(rows, heads, dim, generator=g)).to(torch.bfloat16)
    cache = torch.randn(blocks, page, 1, dim, generator=g).to(torch.bfloat16)
    table = torch.tensor([[4, 1, 3], [0, 2, -1], [5, 5, 5]], dtype=torch.int32)
    visible = torch.tensor([9, 5, 0] if dql == 1 else [8, 9, 5, 4, 0, 2], dtype=torch.int32)
    got = oracle.indexer_scores_decode(q, cache, table, visible, dql, 12)
    for r in range(rows):
        keys = []
        for c in range(int(visible[r])):
            keys.append(cache[int(table[r // dql, c // page]), c % page, 0].float().tolist())
        want = restate.relu_head_scores(q[r].float().tolist(), keys)
        assert got[r, :len(want)].tolist() == pytest.approx(want, rel=1e-5, abs=1e-5)
        assert torch.isnan(got[r, len(want):]).all()


def test_indexer_invariants():
    g = torch.Generator().manual_seed(6)
    q = torch.randn(2, 4, 16, generator=g).to(torch.bfloat16)
    cache = torch.randn(3, 8, 1, 16, generator=g).to(torch.bfloat16)
    table = torch.tensor([[2, 0, 1], [1, 2, 0]], dtype=torch.int32)
    vis = torch.tensor([24, 17], dtype=torch.int32)
    base = oracle.indexer_scores_decode(q, cache, table, vis, 1, 24)
    assert (base[0] >= 0).all() and (base[1, :17] >= 0).all()
    double = oracle.indexer_scores_decode((q.float() * 2).to(torch.bfloat16), cache, table, vis, 1, 24)
    assert torch.equal(double[0], base[0] * 2)                       # positive homogeneity (exact x2)
    zero = oracle.indexer_scores_decode(torch.zeros_like(q), cache, table, vis, 1, 24)
    assert (zero[0] == 0).all()
    # unit vector on dim 3 in one head: score = relu(k[3]) * 16^-0.5
    unit = torch.zeros_like(q)
    unit[:, 0, 3] = 1
    s = oracle.indexer_scores_decode(unit, cache, table, vis, 1, 24)
    keys = torch.stack([cache[int(table[0, c // 8]), c % 8, 0] for c in range(24)]).float()
    assert torch.allclose(s[0], keys[:, 3].clamp_min(0) * 0.25)


def test_indexer_prefill_matches_decode_rows():
    g = torch.Generator().manual_seed(8)
    q = torch.randn(7, 2, 16, generator=g).to(torch.bfloat16)
    cache = torch.randn(4, 4, 1, 16, generator=g).to(torch.bfloat16)
    table = torch.tensor([[3, 1, 0], [2, 0, 1]], dtype=torch.int32)
    qsl = torch.tensor([10, 14, 17], dtype=torch.int32)  # offset base as in a mixed batch
    vis = torch.tensor([1, 2, 3, 4, 0, 5, 12], dtype=torch.int32)
    pre = oracle.indexer_scores_prefill(q, cache, table, qsl, vis, 2, 4, 16)
    for r in range(2, 6):
        req = 0 if r < 4 else 1
        dec = oracle.indexer_scores_decode(q[r:r + 1], cache, table[req:req + 1], vis[r:r + 1], 1, 16)
        n = int(vis[r])
        assert torch.equal(pre[r - 2, :n], dec[0, :n])


# --------------------------------------------------------------------------- attention


def _paged(seq_len, page, hkv, dim, g, pool_extra=3):
    pages = (seq_len + page - 1) // page
    blocks = pages + pool_extra
    perm = torch.randperm(blocks, generator=g)[:pages]
    k = torch.randn(blocks, page, hkv, dim, generator=g).to(torch.bfloat16)
    v = torch.randn(blocks, page, hkv, dim, generator=g).to(torch.bfloat16)
    return k, v, perm.to(torch.int32)[None]


def test_attention_dense_causal_equals_sdpa():
    g = torch.Generator().manual_seed(9)
    seq_len, page, hq, hkv, dim, n_q = 37, 8, 4, 2, 16, 5
    k, v, table = _paged(seq_len, page, hkv, dim, g)
    q = torch.randn(n_q, hq, dim, generator=g).to(torch.bfloat16)
    pos = list(range(seq_len - n_q, seq_len))
    width = seq_len
    idx = torch.full((n_q, width), -1, dtype=torch.int32)
    for i, p in enumerate(pos):
        idx[i, :p + 1] = torch.arange(p + 1, dtype=torch.int32)
    out = oracle.sparse_attention(q, k, v, idx, table, torch.zeros(n_q, dtype=torch.int32))
    # dense reference through SDPA over the contiguous sequence
    tok = torch.arange(seq_len)
    slots_page = table[0, tok // page].long()
    kd = k[slots_page, tok % page].float()  # [L, hkv, D]
    vd = v[slots_page, tok % page].float()
    kd = kd.repeat_interleave(hq // hkv, dim=1).transpose(0, 1)  # [hq, L, D]
    vd = vd.repeat_interleave(hq // hkv, dim=1).transpose(0, 1)
    mask = torch.tensor([[t <= p for t in range(seq_len)] for p in pos])
    ref = torch.nn.functional.scaled_dot_product_attention(
        q.float().transpose(0, 1), kd, vd, attn_mask=mask)  # [hq, n_q, D]
    assert torch.allclose(out, ref.transpose(0, 1), atol=1e-5, rtol=1e-5)


def test_attention_bruteforce_loops_physical():
    g = torch.Generator().manual_seed(10)
    page, hq, hkv, dim = 4, 2, 1, 8
    k = torch.randn(6, page, hkv, dim, generator=g).to(torch.bfloat16)
    v = torch.randn(6, page, hkv, dim, generator=g).to(torch.bfloat16)
    q = torch.randn(2, hq, dim, generator=g).to(torch.bfloat16)
    idx = torch.tensor([[5, 22, -1, 9, 3, 100], [0, 1, 2, 3, 23, 7]], dtype=torch.int32)
    counts = torch.tensor([5, 4], dtype=torch.int32)
    out = oracle.sparse_attention(q, k, v, idx, torch.zeros(1, 1, dtype=torch.int32),
                                  torch.zeros(2, dtype=torch.int32), indices_are_physical=True,
                                  valid_counts=counts)
    for r in range(2):
        slots = [s for s in idx[r, :int(counts[r])].tolist() if 0 <= s < 6 * page]
        keys = [k[s // page, s % page, 0].float().tolist() for s in slots]
        vals = [v[s // page, s % page, 0].float().tolist() for s in slots]
        for h in range(hq):
            want = restate.softmax_attend(q[r, h].float().tolist(), keys, vals)
            assert out[r, h].tolist() == pytest.approx(want, rel=1e-5, abs=1e-5)


def test_attention_special_cases():
    g = torch.Generator().manual_seed(12)
    k = torch.randn(3, 4, 1, 8, generator=g).to(torch.bfloat16)
    v = torch.randn(3, 4, 1, 8, generator=g).to(torch.bfloat16)
    q = torch.randn(1, 2, 8, generator=g).to(torch.bfloat16)
    table = torch.tensor([[2, 0, 1]], dtype=torch.int32)
    t2r = torch.zeros(1, dtype=torch.int32)
    one = oracle.sparse_attention(q, k, v, torch.tensor([[-1, 6, -1]], dtype=torch.int32), table, t2r)
    # logical token 6 -> logical page 1 -> physical page table[0][1] = 0, offset 2
    assert torch.allclose(one[0], v[0, 2, 0].float().expand(2, 8))
    empty = oracle.sparse_attention(q, k, v, torch.tensor([[-1, -1, 99]], dtype=torch.int32), table, t2r)
    assert (empty == 0).all()
    base_idx = torch.tensor([[0, 5, 9, 10]], dtype=torch.int32)
    a = oracle.sparse_attention(q, k, v, base_idx, table, t2r)
    b = oracle.sparse_attention(q, k, v, base_idx[:, [2, 0, 3, 1]], table, t2r)
    assert torch.allclose(a, b, atol=1e-6)                             # order invariance
    dup = oracle.sparse_attention(q, k, v, torch.tensor([[0, 5, 5]], dtype=torch.int32), table, t2r)
    # duplicate slot counts twice == logit bias ln 2 on that token
    k0 = k[2, 0, 0].float(); k5 = k[0, 1, 0].float()
    v0 = v[2, 0, 0].float(); v5 = v[0, 1, 0].float()
    s0 = q[0].float() @ k0 * 8 ** -0.5
    s5 = q[0].float() @ k5 * 8 ** -0.5 + math.log(2)
    w = torch.softmax(torch.stack([s0, s5], -1), -1)
    assert torch.allclose(dup[0], w[:, :1] * v0 + w[:, 1:] * v5, atol=1e-6)
    gate = torch.randn(1, 2, 8, generator=g).to(torch.bfloat16)
    gated = oracle.sparse_attention(q, k, v, base_idx, table, t2r, output_gate=gate)
    assert torch.equal(gated, a.to(torch.bfloat16).float() * torch.sigmoid(gate.float()))


def test_split_merge_identity():
    g = torch.Generator().manual_seed(13)
    k = torch.randn(8, 4, 2, 16, generator=g).to(torch.bfloat16)
    v = torch.randn(8, 4, 2, 16, generator=g).to(torch.bfloat16)
    q = torch.randn(3, 4, 16, generator=g).to(torch.bfloat16)
    idx = torch.randint(-1, 32, (3, 23), generator=g, dtype=torch.int32)
    counts = torch.tensor([23, 7, 0], dtype=torch.int32)
    single = oracle.sparse_attention(q, k, v, idx, torch.zeros(1, 1, dtype=torch.int32),
                                     torch.zeros(3, dtype=torch.int32), indices_are_physical=True,
                                     valid_counts=counts)
    for splits in (1, 2, 3, 5):
        po, pl = oracle.sparse_attention_partials(
            q, k, v, idx, torch.zeros(1, 1, dtype=torch.int32), torch.zeros(3, dtype=torch.int32),
            splits, indices_are_physical=True, valid_counts=counts, block_n=4)
        merged = oracle.merge_splits(po, pl)
        assert torch.allclose(merged, single, atol=1e-5)


# --------------------------------------------------------------------------- selection by rows


def _int_rows(g, shape, lo=-3, hi=3):
    """Small integers (exact in bf16, so index scores are exact in fp32 and in
    double: integer dot products times 16^-0.5 = 0.25)."""
    return torch.randint(lo, hi + 1, shape, generator=g).to(torch.bfloat16)


def _selection_by_rows(q, cache, table, t2r, pos, seq, ratio, k, width, physical=False,
                       main_table=None, main_page=1):
    """Per row, from its own request: visible blocks, every visible key's score
    by explicit loops, rank-counted top-k, column-wise expansion. Written
    without the oracle's decode/prefill split, so it pins that split."""
    page = cache.shape[1]
    rows_out, counts, visible = [], [], []
    main = main_table.tolist() if main_table is not None else [[0]]
    for r in range(q.shape[0]):
        req = int(t2r[r])
        vis = 0 if req < 0 else min((int(pos[r]) + 1) // ratio, int(seq[req]) // ratio)
        keys = [cache[int(table[req, c // page]), c % page, 0].float().tolist() for c in range(vis)]
        scores = restate.relu_head_scores(q[r].float().tolist(), keys)
        ids = restate.topk_by_rank(restate.u32_keys(torch.tensor(scores, dtype=torch.float32)),
                                   vis, k)
        row, count = restate.expand_columns(ids, int(pos[r]), req, seq.tolist(), ratio, width,
                                            physical, main, main_page)
        rows_out.append(row)
        counts.append(count)
        visible.append(vis)
    return rows_out, counts, visible


def _mixed_batch(seed):
    """Two decode requests of two rows each (decode_query_len 2), two ragged
    prefill chunks (5 and 3 tokens), two padding rows (request -1)."""
    g = torch.Generator().manual_seed(seed)
    ratio, cpage, heads, dim = 4, 4, 2, 16
    seq = torch.tensor([30, 21, 40, 9], dtype=torch.int32)
    pos = torch.tensor([28, 29, 19, 20, 35, 36, 37, 38, 39, 6, 7, 8, 0, 3], dtype=torch.int64)
    t2r = torch.tensor([0, 0, 1, 1, 2, 2, 2, 2, 2, 3, 3, 3, -1, -1], dtype=torch.int32)
    qsl = torch.tensor([0, 2, 4, 9, 12], dtype=torch.int32)
    table = torch.randperm(12, generator=g)[:12].view(4, 3).to(torch.int32)
    cache = _int_rows(g, (12, cpage, 1, dim))
    q = _int_rows(g, (pos.numel(), heads, dim))
    main_page = 8
    main_table = torch.randperm(40, generator=g)[:24].view(4, 6).to(torch.int32)
    main_table[1, 2] = -1                       # an unmapped page: its slots are -1
    return dict(q=q, cache=cache, table=table, t2r=t2r, pos=pos, seq=seq, qsl=qsl,
                ratio=ratio, main_table=main_table, main_page=main_page)


@pytest.mark.parametrize("physical", [False, True])
def test_select_paged_tokens_mixed_batch_by_rows(physical):
    """``ops/indexer.py:346-393``: decode rows (two per request) with
    ``page_table[:num_decodes]``, then prefill rows with
    ``page_table[num_decodes:]`` and ``query_start_loc[num_decodes:]``, and
    padding rows, each equal to its own row's selection."""
    b = _mixed_batch(21 + physical)
    k, ratio = 3, b["ratio"]
    width = k * ratio + ratio - 1
    out, counts, visible = oracle.select_paged_tokens(
        b["q"], b["cache"], b["table"], b["t2r"], b["pos"], b["seq"], k * ratio, ratio,
        query_start_loc=b["qsl"], max_query_len=5, max_seq_len=int(b["seq"].max()),
        num_decodes=2, num_decode_tokens=4, decode_query_len=2,
        main_block_table=b["main_table"] if physical else None, main_page_size=b["main_page"])
    want, want_counts, want_vis = _selection_by_rows(
        b["q"], b["cache"], b["table"], b["t2r"], b["pos"], b["seq"], ratio, k, width,
        physical, b["main_table"], b["main_page"])
    assert visible.tolist() == want_vis
    assert max(want_vis) > k                     # rows really select
    for r in range(out.shape[0]):
        assert out[r].tolist() == want[r], r
    if physical:
        assert counts.tolist() == want_counts


def test_decode_step_against_loops():
    """``attention.py:191-214`` -> ``backend.py:39-68`` in uniform decode:
    physical slots and counts equal each row's own selection; the output
    equals explicit softmax loops over the K/V rows at those slots, and
    attention over the same tokens given as logical ids through the block
    table."""
    g = torch.Generator().manual_seed(31)
    rows, ratio, cpage, hq, hkv, dim, page, k = 3, 4, 4, 4, 2, 16, 8, 3
    seq = torch.tensor([37, 26, 44], dtype=torch.int32)
    pos = seq.long() - 1
    table = torch.randperm(12, generator=g)[:9].view(3, 3).to(torch.int32)
    cache = _int_rows(g, (12, cpage, 1, 16))
    q_idx = _int_rows(g, (rows, 2, 16))
    main_table = torch.randperm(24, generator=g)[:18].view(3, 6).to(torch.int32)
    kc = torch.randn(24, page, hkv, dim, generator=g).to(torch.bfloat16)
    vc = torch.randn(24, page, hkv, dim, generator=g).to(torch.bfloat16)
    q = torch.randn(rows, hq, dim, generator=g).to(torch.bfloat16)
    out, idx, counts = oracle.decode_step(q_idx, cache, table, q, kc, vc, main_table, pos, seq,
                                          k * ratio, ratio)
    width = k * ratio + ratio - 1
    t2r = torch.arange(rows, dtype=torch.int32)
    want, want_counts, _ = _selection_by_rows(q_idx, cache, table, t2r, pos, seq, ratio, k,
                                              width, True, main_table, page)
    assert idx.tolist() == want and counts.tolist() == want_counts
    group = hq // hkv
    for r in range(rows):
        slots = [s for s in idx[r, :int(counts[r])].tolist() if s >= 0]
        assert len(slots) == int(counts[r])
        for h in range(hq):
            keys = [kc[s // page, s % page, h // group].float().tolist() for s in slots]
            vals = [vc[s // page, s % page, h // group].float().tolist() for s in slots]
            w = restate.softmax_attend(q[r, h].float().tolist(), keys, vals)
            assert out[r, h].tolist() == pytest.approx(w, rel=1e-5, abs=1e-5)
    # the same tokens as logical ids (inverse of the block table)
    inverse = {int(main_table[r, i]) * page + o: i * page + o
               for r in range(rows) for i in range(6) for o in range(page)}
    logical = torch.tensor([[inverse[s] if s >= 0 else -1 for s in row] for row in idx.tolist()],
                           dtype=torch.int32)
    again = oracle.sparse_attention(q, kc, vc, logical, main_table, t2r)
    assert torch.allclose(again, out, atol=1e-6)
