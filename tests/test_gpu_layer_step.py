"""The QSA layer step through the metadata builder: eager against the oracle
chain, and a HIP graph captured on one decode batch replayed on another."""

import pytest
import torch

import oracle
from qsa_vllm_amd.backend import QSALayerState, YuLanQSAImpl, YuLanQSAIndexer
from qsa_vllm_amd.graph_dispatch import SHORT_DECODE_COLUMNS, decode_logits_columns
from qsa_vllm_amd.layer_step import QSALayerStepGraph, qsa_layer_step
from qsa_vllm_amd.metadata import QSAMetadataBuilder

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
H_IDX, D_IDX, R, HQ, HKV, D, PAGE, CPAGE, RING, TOPK = 8, 128, 16, 16, 2, 128, 16, 16, 16, 256
MAX_POS, MAX_TOKENS, MAX_REQS = 2048, 96, 8


class World:
    """Caches with history, page tables, layer objects and static buffers."""

    def __init__(self, seed):
        g = torch.Generator().manual_seed(seed)
        main_pages, comp_pages = MAX_POS // PAGE, MAX_POS // R // CPAGE
        self.main_table = torch.randperm(MAX_REQS * main_pages + 3, generator=g)[
            :MAX_REQS * main_pages].view(MAX_REQS, main_pages).to(torch.int32)
        self.comp_table = torch.randperm(MAX_REQS * comp_pages + 2, generator=g)[
            :MAX_REQS * comp_pages].view(MAX_REQS, comp_pages).to(torch.int32)
        self.ring_blocks = torch.randperm(MAX_REQS + 2, generator=g)[:MAX_REQS].to(torch.int32)

        def rnd(*shape):
            return (torch.randn(*shape, generator=g) * 0.5).to(torch.bfloat16).to(DEV)

        self.kv = rnd(MAX_REQS * main_pages + 3, PAGE, HKV, 2 * D)
        self.comp = rnd(MAX_REQS * comp_pages + 2, CPAGE, 1, D_IDX)
        self.ring = rnd(MAX_REQS + 2, RING, D_IDX)
        self.indexer = YuLanQSAIndexer(H_IDX, D_IDX, R, TOPK, 64, 1.0e4, 1e-6, MAX_POS + 64,
                                       self.ring, self.comp)
        self.indexer.q_layernorm.weight.data.copy_(rnd(D_IDX) + 1)
        self.indexer.k_layernorm.weight.data.copy_(rnd(D_IDX) + 1)
        self.layer = QSALayerState(self.kv.permute(0, 2, 1, 3), D, MAX_TOKENS, TOPK + R - 1)
        self.impl = YuLanQSAImpl(HQ, HKV, D)
        self.builder = QSAMetadataBuilder(
            compress_ratio=R, main_page_size=PAGE, comp_page_size=CPAGE, ring_size=RING,
            max_num_requests=MAX_REQS, max_num_tokens=MAX_TOKENS, main_table_width=main_pages,
            comp_table_width=comp_pages, device=DEV)
        idx_cols, kv_cols = (H_IDX + 1) * D_IDX, HKV * D
        self.projected = torch.zeros(MAX_TOKENS, idx_cols + 2 * kv_cols + 64, dtype=torch.bfloat16,
                                     device=DEV)
        self.index_qk = self.projected[:, :idx_cols]
        self.main_key = self.projected[:, idx_cols:idx_cols + kv_cols].view(MAX_TOKENS, HKV, D)
        self.main_value = self.projected[:, idx_cols + kv_cols:idx_cols + 2 * kv_cols].view(
            MAX_TOKENS, HKV, D)
        self.query = torch.zeros(MAX_TOKENS, HQ, D, dtype=torch.bfloat16, device=DEV)
        self.output = torch.zeros(MAX_TOKENS + 2, HQ, D, dtype=torch.bfloat16, device=DEV)

    def state(self):
        return [t.clone() for t in (self.kv, self.comp, self.ring)]

    def restore(self, saved):
        for t, s in zip((self.kv, self.comp, self.ring), saved):
            t.copy_(s)

    def fill(self, tokens, seed):
        g = torch.Generator().manual_seed(seed)
        self.projected[:tokens].copy_((torch.randn(tokens, self.projected.shape[1], generator=g)
                                       * 0.5).to(torch.bfloat16))
        self.query[:tokens].copy_(torch.randn(tokens, HQ, D, generator=g).to(torch.bfloat16))

    def build(self, computed, scheduled):
        n = len(scheduled)
        return self.builder.build(computed, scheduled, self.main_table[:n].to(DEV),
                                  self.comp_table[:n].to(DEV), self.ring_blocks[:n])

    def step(self, batch):
        return qsa_layer_step(self.indexer, self.impl, self.layer, batch, self.index_qk,
                              self.main_key, self.main_value, self.query[:batch.num_tokens],
                              self.output)

    def results(self, n):
        return [self.output[:n].clone(), self.layer.topk_indices_buffer[:n].clone(),
                self.layer.topk_counts_buffer[:n].clone()] + self.state()


def test_decode_graph_replay_equals_eager():
    w = World(seed=1)
    start = w.state()
    computed_a = [300, 511, 1000, 47, 1500, 800]
    computed_b = [1203, 15, 640, 959, 1999, 32]
    print("[layer step] capture on batch A", flush=True)
    w.fill(6, seed=10)
    batch = w.build(computed_a, [1] * 6)
    graph = QSALayerStepGraph(w.indexer, w.impl, w.layer, batch, w.index_qk, w.main_key,
                              w.main_value, w.query[:6], w.output, columns=SHORT_DECODE_COLUMNS)
    for computed, seed in ((computed_b, 11), (computed_a, 12)):
        w.restore(start)
        w.fill(6, seed)
        batch = w.build(computed, [1] * 6)
        w.step(batch)
        torch.cuda.synchronize()
        eager = w.results(6)
        w.restore(start)
        w.fill(6, seed)
        batch = w.build(computed, [1] * 6)
        graph.replay(batch)
        torch.cuda.synchronize()
        replayed = w.results(6)
        for a, b in zip(eager, replayed):
            assert torch.equal(a, b)
        print(f"[layer step] replay equals eager for {computed}", flush=True)


def test_mixed_step_against_oracle():
    """Decode requests first, then prefill chunks: logical ids for every row."""
    w = World(seed=2)
    computed = [700, 129, 40, 300]
    scheduled = [1, 1, 33, 20]
    tokens = sum(scheduled)
    w.fill(tokens, seed=3)
    start = w.state()
    batch = w.build(computed, scheduled)
    w.step(batch)
    torch.cuda.synchronize()
    # oracle prepare on the starting state
    from types import SimpleNamespace
    kv0, comp0, ring0 = [t.cpu() for t in start]
    raw = SimpleNamespace(**{k: v.cpu() for k, v in vars(batch.raw).items()})
    comp_meta = SimpleNamespace(slot_mapping=batch.compressed.slot_mapping.cpu(),
                                k_work_metadata=batch.compressed.k_work_metadata.cpu())
    query_o = oracle.prepare(
        w.index_qk[:tokens].cpu(), batch.positions.cpu(), w.indexer.q_layernorm.weight.data.cpu(),
        w.indexer.k_layernorm.weight.data.cpu(), w.indexer.cos_sin_cache.cpu(), 1e-6, raw,
        comp_meta, ring0, comp0, w.main_key[:tokens].cpu(), w.main_value[:tokens].cpu(),
        kv0[..., :D], kv0[..., D:], batch.main.slot_mapping.cpu(), num_index_heads=H_IDX,
        index_head_dim=D_IDX, rotary_dim=64, compress_ratio=R)
    assert torch.equal(w.comp.cpu(), comp0) and torch.equal(w.kv.cpu(), kv0)
    assert torch.equal(w.ring.cpu(), ring0)
    # selection: GPU scores of the oracle's query per part, oracle top-k
    nd = batch.compressed.num_decode_tokens
    cap = w.comp_table.shape[1] * CPAGE
    visible = batch.compressed.visible_blocks
    qd = query_o.to(DEV)
    cols = decode_logits_columns(batch.compressed.max_seq_len, R, cap)
    lg_d = torch.full((nd, cols), float("nan"), device=DEV)
    torch.ops.yulan_qsa_kernels.indexer_decode(qd[:nd], w.comp, batch.compressed.block_table[:nd],
                                               visible[:nd], lg_d, 1)
    from qsa_vllm_amd.graph_dispatch import prefill_logits_width
    width_p = prefill_logits_width(batch.compressed.max_seq_len, R, cap)
    lg_p = torch.full((tokens - nd, width_p), float("nan"), device=DEV)
    torch.ops.yulan_qsa_kernels.indexer_prefill(qd[nd:], w.comp, batch.compressed.block_table[nd:],
                                                batch.compressed.query_start_loc[nd:],
                                                visible[nd:], lg_p, 0, tokens - nd,
                                                batch.compressed.max_query_len)
    W = TOPK + R - 1
    args = (batch.positions.cpu(), batch.compressed.seq_lens.cpu(), batch.token_to_req.cpu())
    i_d, _ = oracle.topk_expand(lg_d.cpu(), visible[:nd].cpu(), args[0][:nd], args[1],
                                args[2][:nd], None, W, R, PAGE, False)
    i_p, _ = oracle.topk_expand(lg_p.cpu(), visible[nd:].cpu(), args[0][nd:], args[1],
                                args[2][nd:], None, W, R, PAGE, False)
    want_idx = torch.cat([i_d, i_p])
    assert torch.equal(w.layer.topk_indices_buffer[:tokens].cpu(), want_idx)
    want = oracle.sparse_attention(w.query[:tokens].cpu(), kv0[..., :D], kv0[..., D:], want_idx,
                                   batch.main.block_table.cpu(), batch.token_to_req.cpu())
    err = (w.output[:tokens].float().cpu() - want).abs()
    print(f"[layer step] mixed: max_abs={err.max().item():.3e} mean_abs={err.mean().item():.3e}",
          flush=True)
    assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3
