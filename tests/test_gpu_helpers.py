"""GPU parity of the ops/qsa.py helpers (block-id expansion, cache row
stores, group pooling) against the oracle: bit-exact."""

import random

import pytest
import torch

import oracle
from qsa_vllm_amd.ops import (expand_qsa_block_indices_cuda, qsa_compress_groups_with_ratio,
                              qsa_store_cache_rows)

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("ratio,page,physical", [(16, 16, True), (16, 16, False), (4, 6, True),
                                                 (8, 4, True), (4, 8, True)])
def test_expand_block_indices_parity(ratio, page, physical):
    rng = random.Random(ratio * 100 + page)
    g = torch.Generator().manual_seed(ratio + page)
    token_topk, rows, nreq = 128, 37, 6
    k = token_topk // ratio
    width = token_topk + ratio - 1
    seq = torch.randint(0, ratio * (k + 6), (nreq,), generator=g, dtype=torch.int32)
    t2r = torch.randint(-1, nreq, (rows,), generator=g, dtype=torch.int32)
    pos = torch.tensor([rng.randint(0, (int(seq[q]) if q >= 0 else 40) + 2) for q in t2r.tolist()])
    blocks = torch.randint(-2, k + 8, (rows, k + 3), generator=g, dtype=torch.int32)
    table = torch.randint(-1, 500, (nreq, int(seq.max()) // page + 2), generator=g,
                          dtype=torch.int32)
    want, want_cnt = oracle.expand_blocks(blocks, pos, seq, t2r, table if physical else None,
                                          width, ratio, page, physical, k)
    out_base = torch.full((rows, width + 5), -7, dtype=torch.int32, device=DEV)
    out = out_base[:, 2:2 + width]                      # strided rows
    cnt = torch.full((rows,), -7, dtype=torch.int32, device=DEV)
    expand_qsa_block_indices_cuda(blocks.to(DEV), pos.to(DEV), seq.to(DEV), t2r.to(DEV), ratio,
                                  token_topk, out,
                                  main_block_table=table.to(DEV) if physical else None,
                                  main_page_size=page, valid_counts_out=cnt)
    assert torch.equal(out.cpu(), want)
    assert torch.equal(cnt.cpu(), want_cnt)
    assert (out_base[:, :2] == -7).all() and (out_base[:, 2 + width:] == -7).all()


def test_store_cache_rows_parity():
    g = torch.Generator().manual_seed(3)
    cache = (torch.randn(9, 16, 1, 136, generator=g)).to(torch.bfloat16)
    rows = (torch.randn(40, 1, 128, generator=g)).to(torch.bfloat16)
    view = cache[..., :128]                              # key part of a wider row
    slots = torch.randperm(9 * 16, generator=g)[:40].to(torch.int64)
    slots[::7] = -1
    slots[3] = 9 * 16 + 5                                # past the cache: skipped
    want = cache.clone()
    oracle.store_cache_rows(want[..., :128], slots, rows)
    got = cache.to(DEV)
    qsa_store_cache_rows(got[..., :128], slots.to(DEV), rows.to(DEV))
    assert torch.equal(got.cpu(), want)


@pytest.mark.parametrize("rope", [False, True])
def test_compress_groups_parity(rope):
    g = torch.Generator().manual_seed(9)
    ratio, S, dim, nreq = 16, 16, 128, 4
    prefix, chunk = [31, 5, 100, 60], [1, 40, 17, 1]
    qsl = [0]
    for c in chunk:
        qsl.append(qsl[-1] + c)
    rows_req = [q for q in range(nreq) for _ in range(chunk[q])] + [-1, 2]
    rows_pos = [prefix[q] + i for q in range(nreq) for i in range(chunk[q])] + [20, 7]
    rows = len(rows_req)
    slots = torch.tensor([(p * 7) % 50 if (p + 1) % ratio == 0 else -1 for p in rows_pos])
    slots[5] = 3                                          # non-boundary row with a slot
    raw = torch.randn(rows, 1, dim, generator=g).to(torch.bfloat16)
    ring = torch.randn(nreq + 2, S, 1, dim, generator=g).to(torch.bfloat16)
    table = torch.tensor([[4], [0], [-1], [2]], dtype=torch.int32)
    raw_pos = torch.randint(0, 1000, (rows, 1, 3), generator=g)
    ring_pos = torch.randint(0, 1000, (nreq + 2, S, 1, 3), generator=g)
    args = [raw, raw_pos, ring, table, torch.tensor(rows_req, dtype=torch.int32),
            torch.tensor(qsl, dtype=torch.int32), torch.tensor(rows_pos), slots, ratio,
            ring_pos if rope else None]
    want_pooled, want_first = oracle.compress_groups(*args)
    dev_args = [a.to(DEV) if isinstance(a, torch.Tensor) else a for a in args]
    pooled, first = qsa_compress_groups_with_ratio(*dev_args)
    assert torch.equal(pooled.cpu(), want_pooled)
    assert torch.equal(first.cpu(), want_first)
