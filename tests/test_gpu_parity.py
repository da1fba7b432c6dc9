"""GPU parity: the HIP kernels (through the C ABI / torch ops) against the CPU oracle.

Bars: top-k indices, expansion and counts bit-exact on identical fp32 scores;
indexer scores within fp32 accumulation error (|err| <= 2e-5 * sum|q*k| * D^-0.5
+ 1e-6); attention within max-abs 2e-2 and mean-abs 2e-3 of the fp32 oracle.
"""

import math

import pytest
import torch

import oracle
from qsa_vllm_amd.ops import (qsa_sparse_paged_attention, select_paged_tokens, topk,
                              topk_expand)
from qsa_vllm_amd.workloads import make_workload

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def _note(msg):
    print(f"[case] {msg}", flush=True)


def _special_scores(rows, cols, g, mode):
    if mode == "random":
        return torch.randn(rows, cols, generator=g) * 10
    if mode == "ties":
        return torch.randint(0, 5, (rows, cols), generator=g).float()
    if mode == "relu":  # nonnegative with exact zeros, like ReLU-summed scores
        return (torch.randn(rows, cols, generator=g) * 4).clamp_min(0)
    if mode == "specials":
        pool = torch.tensor([0.0, -0.0, 1.0, -1.0, float("inf"), float("-inf"), 1e-40, 3.5],
                            dtype=torch.float32)
        s = pool[torch.randint(0, len(pool), (rows, cols), generator=g)]
        nan_bits = torch.tensor([0x7FC00000, 0x7F800001, -4194304], dtype=torch.int32)
        mask = torch.rand(rows, cols, generator=g) < 0.05
        nans = nan_bits[torch.randint(0, 3, (rows, cols), generator=g)].view(torch.float32)
        return torch.where(mask, nans, s)
    raise ValueError(mode)


# Up to 1023 rows, widths past 2048 up to 32768 take the workgroup-per-row
# shape sized by each row's own length (2-16 keys per thread; rows over 16384
# keys in two halves and a merge of their winners); wider rows the partition +
# merge launches.
@pytest.mark.parametrize("cols,k", [(64, 16), (1000, 128), (2048, 128), (4096, 128), (8192, 128),
                                    (16384, 512), (20000, 128), (32768, 2048), (40000, 128),
                                    (70000, 512)])
@pytest.mark.parametrize("mode", ["random", "ties", "relu", "specials"])
def test_topk_bit_exact(cols, k, mode):
    _note(f"topk cols={cols} k={k} mode={mode}")
    g = torch.Generator().manual_seed(cols * 7 + k + len(mode))
    rows = 6 if cols > 16384 else 33
    scores = _special_scores(rows, cols, g, mode)
    lengths = torch.randint(0, cols + 1, (rows,), generator=g, dtype=torch.int32)
    lengths[0], lengths[1], lengths[2] = cols, k, min(cols, k + 1)
    if rows > 5:  # lengths at the per-thread size boundaries of the row-sized shape
        lengths[3], lengths[4], lengths[5] = min(cols, 2048), min(cols, 2049), min(cols, 16385)
    lengths[-1] = -5  # a negative length selects nothing (ids -1), like a length of 0
    want = oracle.topk_ids(scores, lengths, k)
    out = torch.full((rows, k), -7, dtype=torch.int32, device=DEV)
    topk(scores.to(DEV), lengths.to(DEV), out)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), want)


# Seeded random launches over every top-k path: row counts on both sides of
# the throughput switch, widths at the launch-shape boundaries (2048 / 4096 /
# 8192 / 16384 / 32768 and one past each), k from 1 to 512, lengths from -3 to
# the width, every score mode; plain selection and physical expansion.
_SWEEP_COLS = [5, 100, 1000, 2048, 2049, 3000, 4096, 4097, 8192, 9000, 16384, 16385, 32768,
               40000]


@pytest.mark.parametrize("seed", range(48))
def test_topk_random_launches(seed):
    g = torch.Generator().manual_seed(1000 + seed)
    pick = lambda seq: seq[int(torch.randint(0, len(seq), (1,), generator=g))]  # noqa: E731
    cols = pick(_SWEEP_COLS)
    k = pick([1, 16, 64, 128, 512])
    mode = pick(["random", "ties", "relu", "specials"])
    rows = pick([1, 3, 17, 64, 200, 1100])
    rows = max(1, min(rows, 3_000_000 // cols))
    _note(f"topk sweep seed={seed} rows={rows} cols={cols} k={k} mode={mode}")
    scores = _special_scores(rows, cols, g, mode)
    lengths = torch.randint(-3, cols + 1, (rows,), generator=g, dtype=torch.int32)
    lengths[0] = cols
    want = oracle.topk_ids(scores, lengths, k)
    out = torch.full((rows, k), -7, dtype=torch.int32, device=DEV)
    topk(scores.to(DEV), lengths.to(DEV), out)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), want)
    # The same rows expanded to physical slots (ratio 16, page 16), with counts.
    ratio, page = 16, 16
    width = k * ratio + ratio - 1
    vis = lengths.clamp_min(0)
    seq = (vis.long() * ratio + torch.randint(0, ratio, (rows,), generator=g)).to(torch.int32)
    pos = seq.long() - 1
    t2r = torch.arange(rows, dtype=torch.int32)
    table = torch.randint(0, 1 << 20, (rows, cols + 2), generator=g, dtype=torch.int32)
    want_e, want_c = oracle.topk_expand(scores, vis, pos, seq, t2r, table, width, ratio, page, True)
    got_e = torch.full((rows, width), -9, dtype=torch.int32, device=DEV)
    got_c = torch.full((rows,), -9, dtype=torch.int32, device=DEV)
    topk_expand(scores.to(DEV), vis.to(DEV), pos.to(DEV), seq.to(DEV), t2r.to(DEV), got_e, ratio,
                main_block_table=table.to(DEV), main_page_size=page, valid_counts_out=got_c)
    torch.cuda.synchronize()
    assert torch.equal(got_e.cpu(), want_e)
    assert torch.equal(got_c.cpu(), want_c)


# 1024+ rows switch top-k to its throughput launch shapes and row writer.
@pytest.mark.parametrize("cols,ratio,page,physical", [(1000, 16, 16, True), (2048, 16, 16, False),
                                                      (3000, 4, 6, True), (2048, 4, 8, True)])
def test_topk_expand_many_rows(cols, ratio, page, physical):
    _note(f"topk_expand many rows cols={cols} ratio={ratio} page={page} physical={physical}")
    g = torch.Generator().manual_seed(cols + ratio + page)
    rows, k = 1100, 64
    seq, t2r, pos, vis, table, scores = _expand_case(g, rows, cols, ratio, page, k, physical, reqs=9)
    width = k * ratio + ratio - 1
    want, want_counts = oracle.topk_expand(scores, vis, pos, seq, t2r, table, width, ratio, page,
                                           physical)
    out = torch.full((rows, width), -9, dtype=torch.int32, device=DEV)
    counts = torch.full((rows,), -9, dtype=torch.int32, device=DEV)
    topk_expand(scores.to(DEV), vis.to(DEV), pos.to(DEV), seq.to(DEV), t2r.to(DEV), out, ratio,
                main_block_table=table.to(DEV) if physical else None, main_page_size=page,
                valid_counts_out=counts)
    plain = torch.full((rows, k), -9, dtype=torch.int32, device=DEV)
    topk(scores.to(DEV), vis.to(DEV), plain)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), want)
    assert torch.equal(counts.cpu(), want_counts)
    assert torch.equal(plain.cpu(), oracle.topk_ids(scores, vis, k))


def _expand_case(g, rows, cols, ratio, page, k, physical, reqs=5):
    seq = torch.randint(0, cols * ratio + 40, (reqs,), generator=g, dtype=torch.int32)
    t2r = torch.randint(-1, reqs + 1, (rows,), generator=g, dtype=torch.int32)
    t2r[:4] = torch.arange(4, dtype=torch.int32) % reqs
    mapped = (t2r >= 0) & (t2r < reqs)
    sl = torch.where(mapped, seq[t2r.clamp(0, reqs - 1).long()], torch.zeros_like(seq[:1]))
    pos = (torch.rand(rows, generator=g) * (sl.float() + 20)).long()
    # visible blocks of mapped rows; unmapped rows (padding or out-of-range request) see none
    vis = torch.where(mapped, torch.minimum((pos + 1) // ratio, sl.long() // ratio),
                      torch.zeros_like(pos)).to(torch.int32).clamp_max(cols)
    vis[-1] = cols  # a row whose visible count exceeds the token budget
    width = (max(int(seq.max()), 1) + page - 1) // page + 1
    table = torch.randint(0, 1000, (reqs, width), generator=g, dtype=torch.int32)
    table[torch.rand(reqs, width, generator=g) < 0.1] = -1
    scores = (torch.randn(rows, cols, generator=g) * 3).clamp_min(0)
    return seq, t2r, pos, vis, table, scores


@pytest.mark.parametrize("ratio,page,physical", [(16, 16, True), (4, 272, True), (4, 6, True),
                                                 (4, 16, False), (16, 16, False), (1, 16, True)])
@pytest.mark.parametrize("cols,k", [(2048, 128), (9000, 64), (32768, 128), (40000, 128)])
def test_topk_expand_bit_exact(ratio, page, physical, cols, k):
    _note(f"topk_expand ratio={ratio} page={page} physical={physical} cols={cols} k={k}")
    g = torch.Generator().manual_seed(ratio * 1000 + page + cols + physical)
    rows = 8 if cols > 16384 else 40
    seq, t2r, pos, vis, table, scores = _expand_case(g, rows, cols, ratio, page, k, physical)
    if cols == 32768:  # rows over 16384 keys: two halves, then their winners
        vis[-2], vis[-3] = 16385, 30000
    width = k * ratio + ratio - 1
    want, want_counts = oracle.topk_expand(scores, vis, pos, seq, t2r, table, width, ratio, page,
                                           physical)
    # A strided output view checks that the column stride is honoured.
    big = torch.full((rows, 2 * width), -9, dtype=torch.int32, device=DEV)
    out = big[:, ::2]
    counts = torch.full((rows,), -9, dtype=torch.int32, device=DEV)
    topk_expand(scores.to(DEV), vis.to(DEV), pos.to(DEV), seq.to(DEV), t2r.to(DEV), out, ratio,
                main_block_table=table.to(DEV) if physical else None, main_page_size=page,
                valid_counts_out=counts)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), want)
    assert torch.equal(counts.cpu(), want_counts)
    assert (big[:, 1::2] == -9).all()
    # A contiguous output view starting 4 bytes past a 16-byte boundary, with
    # nothing written outside it.
    flat = torch.full((rows * width + 2,), -9, dtype=torch.int32, device=DEV)
    out_c = flat[1:1 + rows * width].view(rows, width)
    topk_expand(scores.to(DEV), vis.to(DEV), pos.to(DEV), seq.to(DEV), t2r.to(DEV), out_c, ratio,
                main_block_table=table.to(DEV) if physical else None, main_page_size=page)
    torch.cuda.synchronize()
    assert torch.equal(out_c.cpu(), want)
    assert flat[0].item() == -9 and flat[-1].item() == -9


def _score_tol(q, keys, dim):
    mag = (q.float().abs() @ keys.float().abs().T).sum(0) * dim ** -0.5
    return 2e-5 * mag + 1e-6


# The last three cases launch at least one wave per CU, which takes the
# eight-tiles-per-wave split; the others take four. Head dim 128 moves the keys
# into LDS (the index cache page is 16 keys), head dim 64 loads them straight
# into the MFMA operand.
# The 64 x 400 case's longest rows need two passes of their waves (rows stride
# over their keys, reusing the wave's LDS region: the grid follows the batch,
# not the logits width). The 520-row case's first 512 rows, launched alone (a
# different program count), must match bit for bit.
@pytest.mark.parametrize("heads,dim,dql,reqs,width", [
    (32, 128, 1, 9, 13), (8, 64, 1, 9, 13), (4, 128, 2, 9, 13), (48, 128, 1, 9, 13),
    (32, 128, 1, 36, 64), (16, 64, 2, 20, 64), (32, 128, 1, 64, 400), (8, 64, 1, 520, 4)])
def test_indexer_decode_parity(heads, dim, dql, reqs, width):
    _note(f"indexer_decode heads={heads} dim={dim} dql={dql} reqs={reqs} width={width}")
    g = torch.Generator().manual_seed(heads + dim + dql + reqs)
    cpage = 16
    rows = reqs * dql
    pool = max(150, reqs * width + 7)
    q = torch.randn(rows, heads, dim, generator=g).to(torch.bfloat16)
    cache = torch.randn(pool, cpage, 1, dim, generator=g).to(torch.bfloat16)
    table = torch.randperm(pool, generator=g)[:reqs * width].view(reqs, width).to(torch.int32)
    vis = torch.randint(0, width * cpage + 1, (rows,), generator=g, dtype=torch.int32)
    vis[0], vis[1] = width * cpage, 0
    cols = width * cpage
    want = oracle.indexer_scores_decode(q, cache, table, vis, dql, cols)
    logits = torch.full((rows, cols), float("nan"), device=DEV)
    torch.ops.yulan_qsa_kernels.indexer_decode(q.to(DEV), cache.to(DEV), table.to(DEV), vis.to(DEV),
                                               logits, dql)
    got = logits.cpu()
    for r in range(rows):
        n = int(vis[r])
        c = torch.arange(n)
        keys = cache[table[r // dql, c // cpage].long(), c % cpage, 0]
        if n:
            tol = _score_tol(q[r], keys, dim)
            assert ((got[r, :n] - want[r, :n]).abs() <= tol).all(), r
        assert torch.isnan(got[r, n:]).all(), "columns beyond visible must stay untouched"
    if rows * ((cols + 127) // 128) >= 256:
        # The first two requests alone take the four-tile split: same bits.
        sub = 2 * dql
        small = torch.full((sub, cols), float("nan"), device=DEV)
        torch.ops.yulan_qsa_kernels.indexer_decode(q[:sub].to(DEV), cache.to(DEV), table[:2].to(DEV),
                                                   vis[:sub].to(DEV), small, dql)
        assert torch.equal(small.cpu().nan_to_num(-7.0), got[:sub].nan_to_num(-7.0))
    if rows > 512:
        part = torch.full((512, cols), float("nan"), device=DEV)
        torch.ops.yulan_qsa_kernels.indexer_decode(q[:512].to(DEV), cache.to(DEV), table.to(DEV),
                                                   vis[:512].to(DEV), part, dql)
        assert torch.equal(part.cpu().nan_to_num(-7.0), got[:512].nan_to_num(-7.0))


def test_indexer_prefill_parity():
    _note("indexer_prefill")
    g = torch.Generator().manual_seed(21)
    heads, dim, cpage = 32, 128, 16
    lens = [37, 1, 70, 20]
    qsl = torch.tensor([5] + [5 + sum(lens[:i + 1]) for i in range(len(lens))], dtype=torch.int32)
    rows = sum(lens)
    width = 6
    q = torch.randn(rows, heads, dim, generator=g).to(torch.bfloat16)
    cache = torch.randn(40, cpage, 1, dim, generator=g).to(torch.bfloat16)
    table = torch.randperm(40, generator=g)[:len(lens) * width].view(len(lens), width).to(torch.int32)
    vis = torch.randint(0, width * cpage + 1, (rows,), generator=g, dtype=torch.int32)
    lw = width * cpage
    for offset, n in [(0, rows), (30, 50)]:
        want = oracle.indexer_scores_prefill(q, cache, table, qsl, vis, offset, n, lw)
        logits = torch.full((n, lw), float("nan"), device=DEV)
        torch.ops.yulan_qsa_kernels.indexer_prefill(q.to(DEV), cache.to(DEV), table.to(DEV),
                                                    qsl.to(DEV), vis.to(DEV), logits, offset, n,
                                                    max(lens))
        got = logits.cpu()
        written = ~torch.isnan(want)
        assert torch.equal(written, ~torch.isnan(got))
        assert torch.allclose(got[written], want[written], rtol=2e-5, atol=2e-4)


@pytest.mark.parametrize("dim,heads", [(128, 32), (64, 20)])
def test_indexer_prefill_many_requests(dim, heads):
    """More than 64 requests (the request search takes several ballots), empty
    requests, 32-row tiles crossing several request boundaries, spans starting
    inside a request, and key-range chunks."""
    _note(f"indexer_prefill many requests dim={dim} heads={heads}")
    g = torch.Generator().manual_seed(23)
    cpage, width = 16, 16
    lens = torch.randint(0, 40, (150,), generator=g)
    lens[torch.rand(150, generator=g) < 0.15] = 0
    lens[3] = 300  # one long request: tiles inside a single request
    nreq = len(lens)
    qsl = torch.zeros(nreq + 1, dtype=torch.int32)
    qsl[1:] = torch.cumsum(lens, 0).to(torch.int32)
    qsl += 7
    rows = int(lens.sum())
    q = torch.randn(rows, heads, dim, generator=g).to(torch.bfloat16)
    blocks = nreq * width
    cache = torch.randn(blocks, cpage, 1, dim, generator=g).to(torch.bfloat16)
    table = torch.randperm(blocks, generator=g).view(nreq, width).to(torch.int32)
    lw = width * cpage
    vis = torch.randint(0, lw + 1, (rows,), generator=g, dtype=torch.int32)
    for offset, n in [(0, rows), (45, 333), (rows - 70, 70), (1, 1)]:
        want = oracle.indexer_scores_prefill(q, cache, table, qsl, vis, offset, n, lw)
        logits = torch.full((n, lw), float("nan"), device=DEV)
        torch.ops.yulan_qsa_kernels.indexer_prefill(q.to(DEV), cache.to(DEV), table.to(DEV),
                                                    qsl.to(DEV), vis.to(DEV), logits, offset, n,
                                                    int(lens.max()))
        got = logits.cpu()
        written = ~torch.isnan(want)
        assert torch.equal(written, ~torch.isnan(got)), (offset, n)
        assert torch.allclose(got[written], want[written], rtol=2e-5, atol=2e-4), (offset, n)


@pytest.mark.parametrize("dim,heads", [(128, 32), (64, 20)])
def test_indexer_prefill_balanced_launch(dim, heads):
    """Launches of more than 128 row tiles score each row tile's whole key
    range in one workgroup (no key chunks). Causal chunks of three requests
    give row tiles of 1 to 8 key tiles; 151 row tiles (the last partial), a
    span starting inside a request, and random visibility."""
    _note(f"indexer_prefill balanced launch dim={dim} heads={heads}")
    g = torch.Generator().manual_seed(29)
    cpage, width = 16, 40
    lens = [1500, 1310, 2000]
    prefix = [0, 3000, 6000]
    nreq = len(lens)
    qsl = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0)), dtype=torch.int32)
    rows = sum(lens)
    q = torch.randn(rows, heads, dim, generator=g).to(torch.bfloat16)
    blocks = nreq * width
    cache = torch.randn(blocks, cpage, 1, dim, generator=g).to(torch.bfloat16)
    table = torch.randperm(blocks, generator=g).view(nreq, width).to(torch.int32)
    lw = width * cpage
    causal = torch.cat([(torch.arange(n) + prefix[r] + 1) // 16 for r, n in enumerate(lens)])
    cases = [(causal.clamp_max(lw).to(torch.int32), 0, rows),
             (causal.clamp_max(lw).to(torch.int32), 600, 4200),
             (torch.randint(0, lw + 1, (rows,), generator=g, dtype=torch.int32), 0, rows)]
    for vis, offset, n in cases:
        want = oracle.indexer_scores_prefill(q, cache, table, qsl, vis, offset, n, lw)
        logits = torch.full((n, lw), float("nan"), device=DEV)
        torch.ops.yulan_qsa_kernels.indexer_prefill(q.to(DEV), cache.to(DEV), table.to(DEV),
                                                    qsl.to(DEV), vis.to(DEV), logits, offset, n,
                                                    max(lens))
        got = logits.cpu()
        written = ~torch.isnan(want)
        assert torch.equal(written, ~torch.isnan(got)), (offset, n)
        assert torch.allclose(got[written], want[written], rtol=2e-5, atol=2e-4), (offset, n)


def _attn_check(got, want, what):
    err = (got.float().cpu() - want).abs()
    _note(f"{what}: max_abs={err.max().item():.3e} mean_abs={err.mean().item():.3e}")
    assert err.max().item() <= MAX_ABS and err.mean().item() <= MEAN_ABS, what


# A whole row is compacted to the keys at or above its bound: one per thread
# up to THREADS of them, two per thread up to 2 x THREADS, staged through LDS
# beyond; a 1024-thread row hands up to 1024 candidates to its lower 512
# threads. Rows whose top keys are `ones` tied maxima scattered over the row put
# the candidate count below, between and above those limits for the 512 x 2
# (1000 columns), 512 x 4 (2048), 1024 x 4 (4096) and 1024 x 8 (8192) shapes.
@pytest.mark.parametrize("cols,ones", [(1000, 100), (1000, 600), (2048, 300), (2048, 700),
                                       (2048, 1100), (4096, 300), (4096, 700), (8192, 300),
                                       (8192, 900), (8192, 1500), (8192, 2500)])
def test_topk_whole_row_candidate_counts(cols, ones):
    _note(f"topk whole-row candidates cols={cols} ones={ones}")
    g = torch.Generator().manual_seed(cols + ones)
    rows, k, ratio, page = 6, 128, 16, 16
    scores = torch.rand(rows, cols, generator=g) * 0.5
    for r in range(rows):
        hot = torch.randperm(cols, generator=g)[:ones]
        scores[r, hot] = 1.0 + (r % 2) * torch.randint(0, 3, (ones,), generator=g).float()
    lengths = torch.full((rows,), cols, dtype=torch.int32)
    lengths[5] = cols // 2
    width = k * ratio + ratio - 1
    seq = lengths.long() * ratio + 7
    pos = seq - 1
    t2r = torch.arange(rows, dtype=torch.int32)
    table = torch.randperm(rows * (cols + 1), generator=g).view(rows, cols + 1).to(torch.int32)
    for physical in (False, True):
        idx = torch.full((rows, width), -9, dtype=torch.int32, device=DEV)
        cnt = torch.full((rows,), -9, dtype=torch.int32, device=DEV)
        topk_expand(scores.to(DEV), lengths.to(DEV), pos.to(DEV), seq.to(torch.int32).to(DEV),
                    t2r.to(DEV), idx, ratio,
                    main_block_table=table.to(DEV) if physical else None, main_page_size=page,
                    valid_counts_out=cnt)
        torch.cuda.synchronize()
        want, want_cnt = oracle.topk_expand(scores, lengths, pos, seq.to(torch.int32), t2r,
                                            table if physical else None, width, ratio, page,
                                            physical)
        assert torch.equal(idx.cpu(), want), f"physical={physical}"
        assert torch.equal(cnt.cpu(), want_cnt)


def _random_physical_indices(g, rows, width, num_blocks, page, counts):
    idx = torch.randint(0, num_blocks * page, (rows, width), generator=g, dtype=torch.int32)
    idx[torch.rand(rows, width, generator=g) < 0.05] = -1
    idx[:, -3:] = num_blocks * page + 5        # out-of-cache slots are invalid
    for r in range(rows):
        idx[r, int(counts[r]):] = -1
    return idx


@pytest.mark.parametrize("hq,hkv,dim", [(16, 2, 128), (8, 1, 128), (4, 4, 128), (32, 2, 128),
                                         (64, 2, 128), (16, 2, 64), (8, 8, 64)])
@pytest.mark.parametrize("splits", [1, 3, 8])
@pytest.mark.parametrize("layout", ["token_major", "head_major"])
def test_attention_physical_parity(hq, hkv, dim, splits, layout):
    _physical_case(hq, hkv, dim, splits, layout, rows=6)


# 64+ (row, head group) pairs switch the kernel to 8-wave workgroups.
@pytest.mark.parametrize("hq,hkv,dim", [(16, 2, 128), (8, 1, 128), (4, 4, 128), (32, 2, 128),
                                         (16, 2, 64), (8, 8, 64)])
@pytest.mark.parametrize("splits", [1, 3])
@pytest.mark.parametrize("layout", ["token_major", "head_major"])
def test_attention_physical_parity_wide_batch(hq, hkv, dim, splits, layout):
    _physical_case(hq, hkv, dim, splits, layout, rows=72)


@pytest.mark.parametrize("hq,hkv,dim", [(16, 2, 128), (4, 4, 128), (8, 8, 64), (16, 4, 64)])
@pytest.mark.parametrize("splits", [1, 2])
def test_attention_physical_parity_grouped_heads(hq, hkv, dim, splits):
    """Batches of a full round of workgroups or more: decode rows then group
    several kv heads per workgroup (at smaller batches each kv head gets its
    own workgroup)."""
    _physical_case(hq, hkv, dim, splits, "token_major", rows=264)


@pytest.mark.parametrize("config,splits", [((64, 1, 4), 1), ((32, 2, 4), 2), ((32, 8, 1), 4),
                                           ((16, 64, 4), 8)])
def test_attention_decode_config_through_plugin_call(config, splits):
    """``qsa_sparse_paged_attention(..., decode_config=...)`` on decode rows:
    the caller's (block_n, target_splits, warps) sets the split count as the
    reference does (ops/qsa.py:643-645) and every count matches the oracle."""
    from qsa_vllm_amd.ops import qsa_sparse_paged_attention
    from qsa_vllm_amd.ops.qsa import choose_num_splits
    _note(f"attention decode_config={config}")
    g = torch.Generator().manual_seed(sum(config))
    hq, hkv, dim, rows, page, num_blocks, width = 16, 2, 128, 12, 16, 40, 200
    kv = torch.randn(num_blocks, page, hkv, 2 * dim, generator=g).to(torch.bfloat16)
    k, v = kv[..., :dim], kv[..., dim:]
    q = torch.randn(rows, hq, dim, generator=g).to(torch.bfloat16)
    counts = torch.tensor([width, 0, 1, 33, 150, 199], dtype=torch.int32).repeat(rows // 6)
    idx = _random_physical_indices(g, rows, width, num_blocks, page, counts)
    table = torch.zeros(1, 1, dtype=torch.int32)
    t2r = torch.zeros(rows, dtype=torch.int32)
    kvd = kv.to(DEV)
    assert choose_num_splits(q, kvd[..., :dim], idx, True, config) == splits
    want = oracle.sparse_attention(q, k, v, idx, table, t2r, indices_are_physical=True,
                                   valid_counts=counts)
    out = qsa_sparse_paged_attention(q.to(DEV), kvd[..., :dim], kvd[..., dim:], idx.to(DEV),
                                     table.to(DEV), t2r.to(DEV), use_decode_kernel=True,
                                     indices_are_physical=True, valid_counts=counts.to(DEV),
                                     decode_config=config)
    torch.cuda.synchronize()
    _attn_check(out, want, f"decode_config={config}")


def _physical_case(hq, hkv, dim, splits, layout, rows):
    _note(f"attention physical hq={hq} hkv={hkv} dim={dim} splits={splits} layout={layout} "
          f"rows={rows}")
    g = torch.Generator().manual_seed(hq * 31 + hkv * 7 + dim + splits + rows)
    page, num_blocks, width = 16, 40, 200
    if layout == "token_major":
        kv = torch.randn(num_blocks, page, hkv, 2 * dim, generator=g).to(torch.bfloat16)
        k, v = kv[..., :dim], kv[..., dim:]
    else:
        kv = torch.randn(num_blocks, hkv, page, 2 * dim, generator=g).to(torch.bfloat16)
        k, v = kv.transpose(1, 2).split(dim, dim=-1)
    q = torch.randn(rows, hq, dim, generator=g).to(torch.bfloat16)
    gate = torch.randn(rows, hq, dim, generator=g).to(torch.bfloat16)
    counts = torch.tensor([width, 0, 1, 33, 150, 199], dtype=torch.int32).repeat(rows // 6)
    idx = _random_physical_indices(g, rows, width, num_blocks, page, counts)
    table = torch.zeros(1, 1, dtype=torch.int32)
    t2r = torch.zeros(rows, dtype=torch.int32)
    kvd = kv.to(DEV)
    if layout == "token_major":
        kd, vd = kvd[..., :dim], kvd[..., dim:]
    else:
        kd, vd = kvd.transpose(1, 2).split(dim, dim=-1)
    for use_gate in (False, True):
        want = oracle.sparse_attention(q, k, v, idx, table, t2r, indices_are_physical=True,
                                       valid_counts=counts, output_gate=gate if use_gate else None)
        out = torch.full((rows, hq, dim), float("nan"), dtype=torch.bfloat16, device=DEV)
        torch.ops.yulan_qsa_kernels.sparse_attention(
            q.to(DEV), kd, vd, idx.to(DEV), table.to(DEV), t2r.to(DEV), out,
            gate.to(DEV) if use_gate else None, counts.to(DEV), True, splits)
        torch.cuda.synchronize()
        _attn_check(out, want, f"gate={use_gate}")
        assert (out[1::6].float() == 0).all(), "a row with no valid slot must be zero"


# Logical (prefill) rows group up to four kv heads per workgroup (NKV = 4, 2
# or 1 by head shape), and with D = 128 each NKV is its own K-into-LDS kernel
# with its own wait counts, so every head shape that picks a different NKV runs
# here: (16, 2) NKV 2, (8, 1) and (32, 2) NKV 1, (4, 4) and (16, 4) NKV 4,
# (64, 2) NKV 1 with 16-head groups, and D = 64 with NKV 2 and 4.
@pytest.mark.parametrize("hq,hkv,dim", [(16, 2, 128), (8, 1, 128), (4, 4, 128), (32, 2, 128),
                                         (16, 4, 128), (64, 2, 128), (16, 2, 64), (8, 8, 64)])
@pytest.mark.parametrize("splits", [1, 4])
@pytest.mark.parametrize("reps", [1, 8])
def test_attention_logical_parity(hq, hkv, dim, splits, reps):
    _note(f"attention logical hq={hq} hkv={hkv} dim={dim} splits={splits} rows={9 * reps}")
    g = torch.Generator().manual_seed(40 + splits + reps + hq * 3 + hkv + dim)
    reqs, page, num_blocks = 3, 16, 30
    k = torch.randn(num_blocks, page, hkv, dim, generator=g).to(torch.bfloat16)
    v = torch.randn(num_blocks, page, hkv, dim, generator=g).to(torch.bfloat16)
    table = torch.randperm(num_blocks, generator=g)[:reqs * 8].view(reqs, 8).to(torch.int32)
    table[1, 5:] = -1
    table[2, 0] = num_blocks + 4             # an out-of-cache page is invalid
    rows, width = 9 * reps, 100
    # padding (-1) and out-of-range request rows repeat every 9 rows
    t2r = torch.tensor([0, 0, 1, 1, 2, 2, -1, 3, 0], dtype=torch.int32).repeat(reps)
    idx = torch.randint(-2, 8 * page + 10, (rows, width), generator=g, dtype=torch.int32)
    q = torch.randn(rows, hq, dim, generator=g).to(torch.bfloat16)
    gate = torch.randn(rows, hq, dim, generator=g).to(torch.bfloat16)
    bad = ((t2r < 0) | (t2r >= reqs)).to(DEV)
    for use_gate in (False, True):
        want = oracle.sparse_attention(q, k, v, idx, table, t2r,
                                       output_gate=gate if use_gate else None)
        out = torch.full((rows, hq, dim), float("nan"), dtype=torch.bfloat16, device=DEV)
        torch.ops.yulan_qsa_kernels.sparse_attention(
            q.to(DEV), k.to(DEV), v.to(DEV), idx.to(DEV), table.to(DEV), t2r.to(DEV), out,
            gate.to(DEV) if use_gate else None, None, False, splits)
        torch.cuda.synchronize()
        _attn_check(out, want, f"logical gate={use_gate}")
        assert (out[bad].float() == 0).all()
    # the plugin's call (the library picks the split count for the shape)
    out = qsa_sparse_paged_attention(q.to(DEV), k.to(DEV), v.to(DEV), idx.to(DEV), table.to(DEV),
                                     t2r.to(DEV))
    torch.cuda.synchronize()
    _attn_check(out, oracle.sparse_attention(q, k, v, idx, table, t2r), "logical, library split")


# Seeded random attention launches: head groupings, head dims, batch sizes on
# both sides of the launch-plan switches, widths, split counts, physical and
# logical indices (with padding rows and invalid entries), both cache layouts
# and the output gate.
_SWEEP_HEADS = [(16, 2, 128), (8, 1, 128), (4, 4, 128), (32, 2, 128), (16, 4, 128), (64, 2, 128),
                (16, 2, 64), (8, 8, 64)]


@pytest.mark.parametrize("seed", range(24))
def test_attention_random_launches(seed):
    g = torch.Generator().manual_seed(2000 + seed)
    pick = lambda seq: seq[int(torch.randint(0, len(seq), (1,), generator=g))]  # noqa: E731
    hq, hkv, dim = pick(_SWEEP_HEADS)
    rows, width = pick([1, 5, 37, 70, 300]), pick([1, 31, 100, 257, 600])
    splits, physical, use_gate = pick([1, 2, 3, 5, 8]), pick([True, False]), pick([True, False])
    layout = pick(["token_major", "head_major"]) if physical else "token_major"
    _note(f"attention sweep seed={seed} hq={hq} hkv={hkv} dim={dim} rows={rows} width={width} "
          f"splits={splits} physical={physical} gate={use_gate} layout={layout}")
    page, num_blocks, reqs = 16, 48, 4
    if layout == "token_major":
        kv = torch.randn(num_blocks, page, hkv, 2 * dim, generator=g).to(torch.bfloat16)
    else:
        kv = torch.randn(num_blocks, hkv, page, 2 * dim, generator=g).to(torch.bfloat16)
    split_kv = lambda t: ((t[..., :dim], t[..., dim:]) if layout == "token_major"  # noqa: E731
                          else t.transpose(1, 2).split(dim, dim=-1))
    k, v = split_kv(kv)
    q = torch.randn(rows, hq, dim, generator=g).to(torch.bfloat16)
    gate = torch.randn(rows, hq, dim, generator=g).to(torch.bfloat16) if use_gate else None
    if physical:
        counts = torch.randint(0, width + 1, (rows,), generator=g, dtype=torch.int32)
        idx = _random_physical_indices(g, rows, width, num_blocks, page, counts)
        table = torch.zeros(1, 1, dtype=torch.int32)
        t2r = torch.zeros(rows, dtype=torch.int32)
    else:
        counts = None
        table = torch.randperm(num_blocks, generator=g)[:reqs * 10].view(reqs, 10).to(torch.int32)
        table[1, 6:] = -1
        t2r = torch.randint(-1, reqs + 1, (rows,), generator=g, dtype=torch.int32)
        idx = torch.randint(-2, 10 * page + 8, (rows, width), generator=g, dtype=torch.int32)
    want = oracle.sparse_attention(q, k, v, idx, table, t2r, indices_are_physical=physical,
                                   valid_counts=counts, output_gate=gate)
    kd, vd = split_kv(kv.to(DEV))
    out = torch.full((rows, hq, dim), float("nan"), dtype=torch.bfloat16, device=DEV)
    torch.ops.yulan_qsa_kernels.sparse_attention(
        q.to(DEV), kd, vd, idx.to(DEV), table.to(DEV), t2r.to(DEV), out,
        gate.to(DEV) if use_gate else None, counts.to(DEV) if physical else None, physical, splits)
    torch.cuda.synchronize()
    _attn_check(out, want, f"seed={seed}")


def test_decode_select_then_attend_small():
    _note("end-to-end small decode (cpu_decode_4k shape)")
    wl = make_workload("cpu_decode_4k", device="cpu")
    s = wl.shape
    d = {n: getattr(wl, n).to(DEV) for n in ("q_index", "index_cache", "index_table", "token_to_req",
                                              "positions", "seq_lens", "query_start_loc", "visible",
                                              "block_table", "q")}
    kv = wl.kv_cache.to(DEV)
    kd, vd = kv[..., :s.head_dim], kv[..., s.head_dim:]
    rows = wl.rows
    out_idx = torch.empty(rows, s.width, dtype=torch.int32, device=DEV)
    counts = torch.empty(rows, dtype=torch.int32, device=DEV)
    select_paged_tokens(d["q_index"], d["index_cache"], d["index_table"], d["token_to_req"],
                        d["positions"], d["seq_lens"], s.token_topk, s.compress_ratio, out_idx,
                        query_start_loc=d["query_start_loc"], max_query_len=1,
                        max_seq_len=wl.max_seq_len, num_decodes=rows, num_decode_tokens=rows,
                        visible_blocks=d["visible"], main_block_table=d["block_table"],
                        main_page_size=s.page_size, valid_counts_out=counts)
    # Recompute the logits the kernel used, then check top-k bit-exact on them.
    cols = oracle.decode_logits_columns(wl.max_seq_len, s.compress_ratio,
                                        wl.index_table.shape[1] * wl.index_cache.shape[1])
    logits = torch.full((rows, cols), float("nan"), device=DEV)
    torch.ops.yulan_qsa_kernels.indexer_decode(d["q_index"], d["index_cache"], d["index_table"],
                                               d["visible"], logits, 1)
    want_logits = oracle.indexer_scores_decode(wl.q_index, wl.index_cache, wl.index_table,
                                               wl.visible, 1, cols)
    n = int(wl.visible.max())
    assert torch.allclose(logits.cpu()[:, :n], want_logits[:, :n], rtol=2e-5, atol=1e-4)
    want_idx, want_counts = oracle.topk_expand(logits.cpu(), wl.visible, wl.positions, wl.seq_lens,
                                               wl.token_to_req, wl.block_table, s.width,
                                               s.compress_ratio, s.page_size, True)
    assert torch.equal(out_idx.cpu(), want_idx)
    assert torch.equal(counts.cpu(), want_counts)
    out = torch.zeros_like(d["q"])
    qsa_sparse_paged_attention(d["q"], kd, vd, out_idx, d["block_table"], d["token_to_req"], out,
                               use_decode_kernel=True, indices_are_physical=True,
                               valid_counts=counts)
    want = oracle.sparse_attention(wl.q, wl.k_cache, wl.v_cache, want_idx, wl.block_table,
                                   wl.token_to_req, indices_are_physical=True,
                                   valid_counts=want_counts)
    _attn_check(out, want, "decode end-to-end")


def test_graph_replay_matches_eager():
    _note("hip graph replay of the decode step")
    wl = make_workload("cpu_decode_4k", device=DEV, batch=16)
    s = wl.shape
    rows = wl.rows
    out_idx = torch.empty(rows, s.width, dtype=torch.int32, device=DEV)
    counts = torch.empty(rows, dtype=torch.int32, device=DEV)
    out = torch.zeros_like(wl.q)

    def step():
        select_paged_tokens(wl.q_index, wl.index_cache, wl.index_table, wl.token_to_req,
                            wl.positions, wl.seq_lens, s.token_topk, s.compress_ratio, out_idx,
                            query_start_loc=wl.query_start_loc, max_query_len=1,
                            max_seq_len=wl.max_seq_len, num_decodes=rows, num_decode_tokens=rows,
                            visible_blocks=wl.visible, main_block_table=wl.block_table,
                            main_page_size=s.page_size, valid_counts_out=counts)
        qsa_sparse_paged_attention(wl.q, wl.k_cache, wl.v_cache, out_idx, wl.block_table,
                                   wl.token_to_req, out, use_decode_kernel=True,
                                   indices_are_physical=True, valid_counts=counts)

    step()
    torch.cuda.synchronize()
    ref_out, ref_idx = out.clone(), out_idx.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for i in range(4):
        out.fill_(float("nan"))
        out_idx.fill_(-5)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_idx, ref_idx), i
        assert torch.equal(out, ref_out), i
