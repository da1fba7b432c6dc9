"""CPU pins of the oracle's block-id expansion and group pooling."""

import random

import torch

import oracle
from tests import restate


def test_expand_blocks_matches_triton_twin_statement():
    rng = random.Random(11)
    for ratio, page, physical in [(4, 8, True), (4, 6, True), (4, 4, False), (16, 16, True),
                                  (8, 4, True)]:
        k, rows, nreq = 5, 9, 4
        width = k * ratio + ratio - 1
        seq = [rng.randint(0, ratio * 12) for _ in range(nreq)]
        table_w = max(seq) // page + 2
        table = [[rng.randint(-1, 40) for _ in range(table_w)] for _ in range(nreq)]
        t2r = [rng.randint(-1, nreq - 1) for _ in range(rows)]
        pos = [rng.randint(0, (seq[q] if q >= 0 else 20) + 3) for q in t2r]
        blocks = [[rng.randint(-2, 14) for _ in range(k + 2)] for _ in range(rows)]
        got, counts = oracle.expand_blocks(
            torch.tensor(blocks, dtype=torch.int32), torch.tensor(pos),
            torch.tensor(seq, dtype=torch.int32), torch.tensor(t2r, dtype=torch.int32),
            torch.tensor(table, dtype=torch.int32) if physical else None, width, ratio, page,
            physical, k)
        for r in range(rows):
            want, cnt = restate.expand_columns(blocks[r][:k], pos[r], t2r[r], seq, ratio, width,
                                               physical, table, page)
            assert got[r].tolist() == want, (ratio, page, physical, r)
            assert int(counts[r]) == cnt


def test_compress_groups_matches_position_walk():
    g = torch.Generator().manual_seed(4)
    rng = random.Random(4)
    ratio, S, dim = 4, 6, 64
    # three requests: one decode token, two chunks; one padding row (request -1)
    prefix, chunk = [9, 2, 13], [1, 7, 5]
    qsl = [0]
    for c in chunk:
        qsl.append(qsl[-1] + c)
    rows_req = [q for q in range(3) for _ in range(chunk[q])] + [-1]
    rows_pos = [prefix[q] + i for q in range(3) for i in range(chunk[q])] + [5]
    rows_slot = [rng.choice([-1, rng.randint(0, 30)]) if (p + 1) % ratio == 0 else -1
                 for p in rows_pos]
    rows_slot[3] = 7                      # a slot on a non-boundary row still pools
    rows = len(rows_req)
    raw = (torch.randn(rows, 1, dim, generator=g)).to(torch.bfloat16)
    ring = (torch.randn(5, S, 1, dim, generator=g)).to(torch.bfloat16)
    blocks = [3, -1, 0]
    raw_pos = torch.randint(0, 100, (rows, 1, 3), generator=g)
    ring_pos = torch.randint(0, 100, (5, S, 1, 3), generator=g)
    for rope in (False, True):
        pooled, firsts = oracle.compress_groups(
            raw, raw_pos, ring, torch.tensor(blocks, dtype=torch.int32).view(3, 1),
            torch.tensor(rows_req, dtype=torch.int32), torch.tensor(qsl, dtype=torch.int32),
            torch.tensor(rows_pos), torch.tensor(rows_slot), ratio,
            ring_pos if rope else None)
        want, want_first = restate.pool_rows(
            rows_req, rows_pos, rows_slot, qsl, blocks,
            [[ring[b, s, 0].float().tolist() for s in range(S)] for b in range(5)],
            [raw[r, 0].float().tolist() for r in range(rows)], ratio, S,
            raw_pos[:, 0].tolist() if rope else None,
            [[ring_pos[b, s, 0].tolist() for s in range(S)] for b in range(5)] if rope else None)
        assert pooled[:, 0].float().tolist() == want
        assert firsts.tolist() == want_first


def test_store_cache_rows_closed_form():
    cache = torch.zeros(3, 4, 1, 8, dtype=torch.bfloat16)
    rows = torch.arange(5 * 8, dtype=torch.float32).view(5, 8).to(torch.bfloat16)
    slots = torch.tensor([5, -1, 11, 12, 0])          # 12 is past 3 x 4 slots
    oracle.store_cache_rows(cache, slots, rows)
    flat = cache.view(12, 8)
    assert torch.equal(flat[5], rows[0]) and torch.equal(flat[11], rows[2])
    assert torch.equal(flat[0], rows[4])
    assert int((flat.abs().sum(1) > 0).sum()) == 2 + (rows[4].abs().sum() > 0)
