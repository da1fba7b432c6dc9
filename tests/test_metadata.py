"""QSAMetadataBuilder against a plain-Python statement of every field (CPU)."""

import random

import pytest
import torch

from qsa_vllm_amd.metadata import QSAMetadataBuilder


def _expected(computed, scheduled, main_table, comp_table, ring_blocks, R, page, cpage, ring,
              dql=1):
    tokens = []
    for q, (c, n) in enumerate(zip(computed, scheduled)):
        for i in range(n):
            tokens.append((q, c + i))
    seq = [c + n for c, n in zip(computed, scheduled)]
    main, raw, comp, vis = [], [], [], []
    for q, p in tokens:
        row = main_table[q]
        pg = row[p // page] if p // page < len(row) else -1
        main.append(pg * page + p % page if pg >= 0 else -1)
        raw.append(ring_blocks[q] * ring + p % ring if ring_blocks[q] >= 0 else -1)
        if (p + 1) % R == 0:
            g = (p + 1) // R - 1
            crow = comp_table[q]
            cp = crow[g // cpage] if g // cpage < len(crow) else -1
            comp.append(cp * cpage + g % cpage if cp >= 0 else -1)
        else:
            comp.append(-1)
        vis.append(min((p + 1) // R, seq[q] // R))
    work = []
    for q, (c, n) in enumerate(zip(computed, scheduled)):
        closed = sum(1 for p in range(c, c + n) if (p + 1) % R == 0)
        work += [[q, w] for w in range(max(closed, 1))]
    decodes = 0
    while decodes < len(scheduled) and scheduled[decodes] == dql:
        decodes += 1
    return tokens, seq, main, raw, comp, vis, work, decodes


def _table(rng, rows, width, pool):
    t = [[rng.randrange(pool) for _ in range(width)] for _ in range(rows)]
    for r in t:
        r[rng.randrange(width)] = -1
    return t


@pytest.mark.parametrize("dql", [1, 2, 3])
def test_builder_matches_plain_statement(dql):
    rng = random.Random(7 + dql)
    R, page, cpage, ring = 4, 4, 2, 4
    b = QSAMetadataBuilder(compress_ratio=R, main_page_size=page, comp_page_size=cpage,
                           ring_size=ring, max_num_requests=8, max_num_tokens=96,
                           main_table_width=12, comp_table_width=8, device="cpu")
    for trial in range(6):
        nreq = rng.randint(1, 8)
        ndec = rng.randint(0, nreq)
        scheduled = [dql] * ndec + [rng.randint(1, 15) for _ in range(nreq - ndec)]
        computed = [rng.randint(0, 30) for _ in range(nreq)]
        main_table = _table(rng, nreq, 12, 50)
        comp_table = _table(rng, nreq, 5, 20)
        ring_blocks = [rng.randint(-1, 9) for _ in range(nreq)]
        batch = b.build(computed, scheduled, torch.tensor(main_table, dtype=torch.int32),
                        torch.tensor(comp_table, dtype=torch.int32), ring_blocks,
                        decode_query_len=dql)
        tokens, seq, main, raw, comp, vis, work, decodes = _expected(
            computed, scheduled, main_table, comp_table, ring_blocks, R, page, cpage, ring, dql)
        assert batch.num_tokens == len(tokens)
        assert batch.positions.tolist() == [p for _, p in tokens]
        assert batch.token_to_req.tolist() == [q for q, _ in tokens]
        assert batch.compressed.seq_lens.tolist() == seq
        assert batch.main.slot_mapping.tolist() == main, trial
        assert batch.raw.slot_mapping.tolist() == raw, trial
        assert batch.compressed.slot_mapping.tolist() == comp, trial
        assert batch.compressed.visible_blocks.tolist() == vis
        kw = batch.compressed.k_work_metadata.tolist()
        assert kw[:len(work)] == work
        assert all(item == [-1, 0] for item in kw[len(work):])
        assert batch.compressed.num_decodes == decodes
        assert batch.compressed.num_decode_tokens == decodes * dql
        assert batch.compressed.decode_query_len == dql
        # decode rows come first: request i owns rows [i * dql, (i + 1) * dql)
        assert batch.token_to_req.tolist()[:decodes * dql] == [
            i for i in range(decodes) for _ in range(dql)]
        assert batch.main.max_query_len == max(scheduled)
        assert batch.raw.query_start_loc.tolist()[-1] == len(tokens)


def test_builder_rejects_oversized_batches():
    b = QSAMetadataBuilder(compress_ratio=4, main_page_size=4, comp_page_size=2, ring_size=4,
                           max_num_requests=2, max_num_tokens=8, main_table_width=4,
                           comp_table_width=4, device="cpu")
    t = torch.zeros(3, 4, dtype=torch.int32)
    for computed, scheduled in (([0, 0, 0], [1, 1, 1]), ([0, 0], [5, 5]), ([0], [0])):
        try:
            b.build(computed, scheduled, t, t, [0, 0, 0])
        except ValueError:
            continue
        raise AssertionError((computed, scheduled))
