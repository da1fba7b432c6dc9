"""The hybrid decoder step on the GPU against the CPU oracle.

A small model (GDN and QSA layers at the serving head shapes, small hidden
size) steps one mixed batch: decode requests, then ragged prefill chunks. It
runs twice: with a top-k budget of 2048 tokens, which every context stays
below (every QSA row attends over its whole causal context), and with a
budget of 256 tokens, which most rows exceed (the QSA layers really select).
Each layer is checked on the GPU layer's own inputs (so rounding does not
accumulate across layers): the QSA selection bit-exact against the oracle's
top-k on the indexer kernel's logits of the layer's prepared index queries,
those logits against the oracle's scores, and the layer's output against the
oracle's attention over the selection; then the final norm and LM head.

The full-size model (32 layers, hidden 4096) on the serving batch of 8304
tokens is checked by properties: finite logits, every QSA layer's selection
against the closed-form counts and row invariants, top-k bit-exact on sampled
rows of one QSA layer, and the decode graph's replay equal to eager."""

import numpy as np
import pytest
import torch

import oracle
import qsa_vllm_amd.backend as backend_module
from oracle import hybrid as H
from qsa_vllm_amd.graph_dispatch import decode_logits_columns, prefill_logits_width
from qsa_vllm_amd.hybrid import (GatedDeltaNet, HybridBatchBuilder, HybridConfig, HybridDecodeGraph,
                                 _Init, make_hybrid_workload, make_serving_hybrid_workload)
from qsa_vllm_amd.ops import hybrid_layers as L
from tests.selection_checks import logical_invariants

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

CFG = HybridConfig(num_layers=4, hidden_size=512, vocab_size=512, tp_size=2, num_heads=32,
                   num_kv_heads=4, head_dim=128, intermediate_size=1024, linear_num_key_heads=4,
                   linear_num_value_heads=8, indexer_heads=8, token_topk=2048, init_std=0.05)
# Top-k 256 tokens = 16 blocks of 16: rows past position 271 select.
CFG_SELECT = HybridConfig(num_layers=4, hidden_size=512, vocab_size=512, tp_size=2, num_heads=32,
                          num_kv_heads=4, head_dim=128, intermediate_size=1024,
                          linear_num_key_heads=4, linear_num_value_heads=8, indexer_heads=8,
                          token_topk=256, init_std=0.05)


def _workload(seed, cfg=CFG):
    return make_hybrid_workload(cfg, decode_lens=[700, 1500, 33, 260], chunk_prefixes=[0, 300, 1000],
                                chunk=100, device=DEV, seed=seed, state_std=0.05)


def _cpu(t):
    return t.detach().cpu()


def _norm_args(n):
    return (_cpu(n.weight), _cpu(n.gate_down), _cpu(n.gate_up), _cpu(n.gate_up_bias), CFG.rms_norm_eps)


def _close(got, want, what, rel_max=0.03, rel_mean=3e-3):
    got, want = got.double().cpu(), want.double().cpu()
    err = (got - want).abs()
    scale = want.abs().max().item()
    print(f"[hybrid] {what}: max_err={err.max().item():.3e} mean_err={err.mean().item():.3e} "
          f"scale={scale:.3e}", flush=True)
    assert err.max().item() <= rel_max * scale and err.mean().item() <= rel_mean * scale, what


def _sequences(wl):
    starts = np.concatenate(([0], np.cumsum(wl.scheduled)[:-1]))
    return [(list(range(int(s), int(s) + n)), int(slot))
            for s, n, slot in zip(starts, wl.scheduled, wl.state_slots)]


def _oracle_qsa(mixer, x, batch, kv0, indices):
    """Projection, K/V writes, attention over ``indices`` (logical token ids)
    with the output gate, o_proj."""
    qkv = H.bf16(x.double() @ _cpu(mixer.qkv_weight).double().T + _cpu(mixer.qkv_bias).double())
    query, gate, key, value, _ = H.qsa_projection_split(qkv, mixer.heads, mixer.kv_heads,
                                                        mixer.head_dim, mixer.index_size)
    kv = kv0.clone()
    page = kv.shape[1]
    d = mixer.head_dim
    for t, slot in enumerate(_cpu(batch.qsa.main.slot_mapping).tolist()):
        kv[slot // page, slot % page, :, :d] = key[t]
        kv[slot // page, slot % page, :, d:] = value[t]
    core = oracle.sparse_attention(query.contiguous(), kv[..., :d], kv[..., d:], indices,
                                   _cpu(batch.qsa.main.block_table), _cpu(batch.qsa.token_to_req),
                                   output_gate=gate.contiguous())
    return H.bf16(H.bf16(core).reshape(x.shape[0], -1).double() @ _cpu(mixer.o_proj).double().T), kv


def _record_index_queries(monkeypatch):
    """Keeps a copy of each QSA layer's prepared index queries (the input of
    its selection) as the layer runs."""
    seen = []
    select = backend_module.select_for_layer

    def recording(index_query, *args, **kwargs):
        seen.append(index_query.clone())
        return select(index_query, *args, **kwargs)

    monkeypatch.setattr(backend_module, "select_for_layer", recording)
    return seen


def _kernel_logits(index_query, comp_cache, md, cfg):
    """The indexer kernels' logits for a batch's rows, as select_paged_tokens
    computes them: decode rows first (decode width class), then prefill rows
    (prefill width). Returns [(rows, logits on the device)]."""
    n = index_query.shape[0]
    nd, nreq_d = md.num_decode_tokens, md.num_decodes
    capacity = md.block_table.shape[1] * comp_cache.shape[1]
    parts = []
    if nd:
        cols = decode_logits_columns(md.max_seq_len, cfg.compress_ratio, capacity)
        lg = torch.full((nd, cols), float("nan"), device=DEV)
        torch.ops.yulan_qsa_kernels.indexer_decode(index_query[:nd], comp_cache,
                                                   md.block_table[:nreq_d],
                                                   md.visible_blocks[:nd], lg, 1)
        parts.append((slice(0, nd), lg))
    if nd < n:
        width = prefill_logits_width(md.max_seq_len, cfg.compress_ratio, capacity)
        lg = torch.full((n - nd, width), float("nan"), device=DEV)
        torch.ops.yulan_qsa_kernels.indexer_prefill(index_query[nd:], comp_cache,
                                                    md.block_table[nreq_d:],
                                                    md.query_start_loc[nreq_d:],
                                                    md.visible_blocks[nd:], lg, 0, n - nd,
                                                    md.max_query_len)
        parts.append((slice(nd, n), lg))
    return parts


def _check_selection(i, mixer, batch, index_query, cfg, rows_checked=None):
    """The layer's selection (logical ids in a mixed batch) bit-exact against
    the oracle's top-k/expansion on the kernel's logits of the layer's own
    index queries, and those logits against the oracle's scores, on
    ``rows_checked`` (default: every row). Returns the selection (CPU)."""
    md = batch.qsa.compressed
    n = batch.num_tokens
    comp = mixer.indexer.compressed_key_cache
    got = _cpu(mixer.layer.topk_indices_buffer[:n])
    vis, pos = _cpu(md.visible_blocks), _cpu(md.logical_positions)
    seq, t2r = _cpu(md.seq_lens), _cpu(md.token_to_req)
    table, qsl = _cpu(md.block_table), _cpu(md.query_start_loc)
    comp_cpu, iq = _cpu(comp), _cpu(index_query)
    nd, nreq_d = md.num_decode_tokens, md.num_decodes
    for rows, lg in _kernel_logits(index_query, comp, md, cfg):
        sel = torch.arange(rows.start, rows.stop)
        if rows_checked is not None:
            sel = sel[torch.isin(sel, rows_checked)]
        logits = _cpu(lg)[sel - rows.start]
        if rows.start == 0:   # decode row r belongs to request r
            want = oracle.indexer_scores_decode(iq[sel], comp_cpu, table[sel], vis[sel], 1,
                                                logits.shape[1])
        else:
            want = torch.cat([oracle.indexer_scores_prefill(iq[nd:], comp_cpu, table[nreq_d:],
                                                            qsl[nreq_d:], vis[nd:], int(r) - nd,
                                                            1, logits.shape[1])
                              for r in sel])
        written = ~torch.isnan(want)
        assert torch.equal(written, ~torch.isnan(logits)), f"layer {i} logits written"
        assert torch.allclose(logits[written], want[written], rtol=2e-5, atol=1e-4), \
            f"layer {i} logits"
        want_idx, _ = oracle.topk_expand(logits, vis[sel], pos[sel], seq, t2r[sel],
                                         torch.zeros(1, 1, dtype=torch.int32), cfg.output_width,
                                         cfg.compress_ratio, cfg.page_size, False)
        assert torch.equal(got[sel], want_idx), f"layer {i} selection"
    return got


def _gdn_params(m):
    return {"in_proj_qkvz": _cpu(m.in_proj_qkvz), "in_proj_ba": _cpu(m.in_proj_ba),
            "conv_weight": _cpu(m.conv_weight), "A_log": _cpu(m.A_log),
            "dt_bias": _cpu(m.dt_bias), "norm_weight": _cpu(m.norm_weight),
            "out_proj": _cpu(m.out_proj)}


@pytest.mark.parametrize("cfg", [CFG, CFG_SELECT], ids=["dense", "selecting"])
def test_hybrid_step_layers_against_oracle(cfg, monkeypatch):
    wl = _workload(seed=5, cfg=cfg)
    model = wl.model
    batch = wl.build()
    torch.cuda.synchronize()
    print(f"[hybrid] token_topk={cfg.token_topk} tokens={wl.num_tokens} "
          f"decodes={batch.num_decode_tokens} layers={[l.kind for l in model.layers]}", flush=True)
    index_queries = _record_index_queries(monkeypatch)
    hidden, residual = model.embed(batch.token_ids), None
    assert torch.equal(_cpu(hidden), _cpu(model.embed_tokens)[torch.as_tensor(wl.token_ids)])
    positions = _cpu(batch.qsa.positions)
    for i, layer in enumerate(model.layers):
        x_in = _cpu(hidden)
        r_in = None if residual is None else _cpu(residual)
        mixer = layer.mixer
        if layer.kind == "linear_attention":
            conv0, ssm0 = _cpu(mixer.conv_state).clone(), _cpu(mixer.ssm_state).clone()
        else:
            kv0 = _cpu(mixer.layer.kv_cache.permute(0, 2, 1, 3))
        hidden, residual = layer(hidden, residual, batch)
        torch.cuda.synchronize()
        # oracle on the same inputs
        if r_in is None:
            n, res = H.gated_norm(x_in, None, *_norm_args(layer.input_layernorm))
            res = x_in
        else:
            n, res = H.gated_norm(x_in, r_in, *_norm_args(layer.input_layernorm))
        if layer.kind == "linear_attention":
            mixed = H.gdn_mixer(n, _gdn_params(mixer), conv0, ssm0, _sequences(wl),
                                key_heads=mixer.hk, value_heads=mixer.hv, key_dim=mixer.dk,
                                value_dim=mixer.dv, eps=CFG.rms_norm_eps)
            # the conv state holds projection outputs: rounding-level differences
            _close(_cpu(mixer.conv_state), conv0, f"layer {i} conv state", 1e-2, 1e-4)
            _close(_cpu(mixer.ssm_state), ssm0, f"layer {i} gdn state", 1e-2, 1e-3)
        else:
            selection = _check_selection(i, mixer, batch, index_queries.pop(0), cfg)
            counts = (selection >= 0).sum(1)
            if cfg.token_topk >= 2048:
                # every row attended over its whole causal context
                assert torch.equal(counts, positions + 1), f"layer {i} selection"
            else:
                selecting = counts < positions + 1
                print(f"[hybrid] layer {i}: {int(selecting.sum())} of {len(counts)} rows select",
                      flush=True)
                assert int(selecting.sum()) > len(counts) // 2, "most rows should select"
            mixed, kv = _oracle_qsa(mixer, n, batch, kv0, selection)
            slots = _cpu(batch.qsa.main.slot_mapping).long()
            page = kv.shape[1]
            got_kv = _cpu(mixer.layer.kv_cache.permute(0, 2, 1, 3))
            _close(got_kv[slots // page, slots % page], kv[slots // page, slots % page],
                   f"layer {i} written K/V rows", 1e-2, 1e-3)
            got_kv[slots // page, slots % page] = kv[slots // page, slots % page]
            assert torch.equal(got_kv, kv), f"layer {i} K/V rows outside the batch's slots"
        n2, res2 = H.gated_norm(mixed, res, *_norm_args(layer.post_attention_layernorm))
        out = H.swiglu(n2, _cpu(layer.mlp.gate_up_proj), _cpu(layer.mlp.down_proj))
        _close(_cpu(residual), res2, f"layer {i} ({layer.kind}) residual")
        _close(_cpu(hidden), out, f"layer {i} ({layer.kind}) output")
    assert not index_queries
    h_in, r_in = _cpu(hidden), _cpu(residual)   # the final norm adds into residual in place
    logits = model.logits(hidden, residual, batch)
    final, _ = H.gated_norm(h_in, r_in, *_norm_args(model.norm))
    rows = _cpu(batch.logits_rows)
    want = H.bf16(final[rows].double() @ _cpu(model.lm_head).double().T)
    _close(_cpu(logits), want, "logits")


def test_hybrid_forward_matches_layerwise_run():
    a, b = _workload(seed=6), _workload(seed=6)
    batch_a, batch_b = a.build(), b.build()
    logits_a = a.model.forward(batch_a)
    hidden, residual = b.model.embed(batch_b.token_ids), None
    for layer in b.model.layers:
        hidden, residual = layer(hidden, residual, batch_b)
    logits_b = b.model.logits(hidden, residual, batch_b)
    torch.cuda.synchronize()
    assert torch.equal(logits_a, logits_b)
    for la, lb in zip(a.model.layers, b.model.layers):
        if la.kind == "linear_attention":
            assert torch.equal(la.mixer.ssm_state, lb.mixer.ssm_state)
            assert torch.equal(la.mixer.conv_state, lb.mixer.conv_state)
        else:
            assert torch.equal(la.mixer.layer.kv_cache, lb.mixer.layer.kv_cache)


def _bf16(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


# Under 1024 rows the library takes its small-batch path (three launches over
# column slices); from 1024 rows the fused 16-token-tile kernel.
@pytest.mark.parametrize("rows,hidden,residual", [(37, 512, False), (37, 512, True),
                                                   (5, 4096, True), (130, 2048, True),
                                                   (1030, 512, False), (1100, 4096, True)])
def test_gated_norm_kernel_against_oracle(rows, hidden, residual):
    x = _bf16((rows, hidden), 1, 2.0)
    res = _bf16((rows, hidden), 2) if residual else None
    w = (1 + 0.3 * _bf16((hidden,), 3).float()).to(torch.bfloat16)
    down, up, bias = _bf16((16, hidden), 4, 0.05), _bf16((hidden, 16), 5, 0.3), _bf16((hidden,), 6, 0.5)
    print(f"[hybrid] gated_norm rows={rows} hidden={hidden} residual={residual}", flush=True)
    res_dev = res.to(DEV) if residual else None
    out, res_out = L.gated_norm(x.to(DEV), res_dev, w.to(DEV), down.to(DEV), up.to(DEV),
                                bias.to(DEV), 1e-6)
    torch.cuda.synchronize()
    want, want_res = H.gated_norm(x, res, w, down, up, bias, 1e-6)
    if residual:
        assert torch.equal(res_out.cpu(), want_res)      # bf16(x + r) is exact
        assert res_out.data_ptr() == res_dev.data_ptr()  # in place
    _close(out.cpu(), want, "gated_norm", 0.02, 2e-3)


def test_silu_mul_kernel_against_oracle():
    gu = _bf16((33, 2 * 5632), 7, 2.0)
    got = L.silu_mul(gu.to(DEV)).cpu()
    i = 5632
    want = H.bf16(torch.nn.functional.silu(gu[:, :i].double()) * gu[:, i:].double())
    diff = (got.float() - want.float()).abs()
    # fp32 arithmetic vs float64: at most one bf16 unit apart
    assert (diff <= want.float().abs() * 2 ** -7 + 1e-30).all()
    assert (got == want).float().mean() > 0.99


def _gdn_setup(seed, slots, key_heads=2, value_heads=4):
    cfg = HybridConfig(num_layers=1, hidden_size=512, tp_size=1, vocab_size=64,
                       linear_num_key_heads=key_heads, linear_num_value_heads=value_heads)
    init = _Init(DEV, seed, 0.05)
    mixer = GatedDeltaNet(cfg, init, num_slots=slots, state_std=0.05)
    mixer.norm_weight = (1 + 0.2 * _bf16((128,), seed).float()).to(torch.bfloat16).to(DEV)
    builder = HybridBatchBuilder(cfg, max_requests=8, max_tokens=256, main_table_width=64,
                                 comp_table_width=8, device=DEV)
    return cfg, mixer, builder


def _gdn_step(mixer, builder, computed, scheduled, slots, seed):
    n = len(scheduled)
    tables = (torch.zeros(n, 64, dtype=torch.int32, device=DEV),
              torch.zeros(n, 8, dtype=torch.int32, device=DEV))
    batch = builder.build(computed, scheduled, [0] * sum(scheduled), *tables,
                          torch.arange(n, dtype=torch.int32), slots)
    x = _bf16((sum(scheduled), 512), seed)
    conv0, ssm0 = _cpu(mixer.conv_state).clone(), _cpu(mixer.ssm_state).clone()
    got = mixer(x.to(DEV), batch)
    torch.cuda.synchronize()
    starts = np.concatenate(([0], np.cumsum(scheduled)[:-1]))
    seqs = [(list(range(int(st), int(st) + k)), int(sl))
            for st, k, sl in zip(starts, scheduled, slots) if 0 <= sl < conv0.shape[0]]
    want = H.gdn_mixer(x, _gdn_params(mixer), conv0, ssm0, seqs, key_heads=mixer.hk,
                       value_heads=mixer.hv, key_dim=128, value_dim=128, eps=1e-6)
    return got, want, conv0, ssm0


# 6 value heads: the projection's row count (qkvz + 2 * 6 gate rows) is not a
# multiple of 8 without the weight's zero padding rows.
@pytest.mark.parametrize("key_heads,value_heads", [(2, 4), (2, 6)])
def test_gdn_mixer_prefill_then_decode_against_oracle(key_heads, value_heads):
    _, mixer, builder = _gdn_setup(seed=21, slots=6, key_heads=key_heads,
                                   value_heads=value_heads)
    assert mixer.in_proj.stride(0) % 8 == 0 and mixer.in_proj.shape[0] % 8 == 0
    # step 1: ragged prefill chunks (one shorter than the conv width) + decodes
    print("[hybrid] gdn step 1", flush=True)
    got, want, conv, ssm = _gdn_step(mixer, builder, [9, 0, 40, 5, 2], [1, 1, 70, 2, 33],
                                     [4, 0, 2, 5, 1], seed=22)
    _close(got.cpu(), want, "gdn step 1 output")
    _close(_cpu(mixer.conv_state), conv, "gdn step 1 conv state", 1e-2, 1e-4)
    _close(_cpu(mixer.ssm_state), ssm, "gdn step 1 state", 1e-2, 1e-3)
    # step 2: every sequence decodes one token from the states just written
    print("[hybrid] gdn step 2", flush=True)
    got, want, conv, ssm = _gdn_step(mixer, builder, [10, 1, 110, 7, 35], [1, 1, 1, 1, 1],
                                     [4, 0, 2, 5, 1], seed=23)
    _close(got.cpu(), want, "gdn step 2 output")
    _close(_cpu(mixer.ssm_state), ssm, "gdn step 2 state", 1e-2, 1e-3)


def test_gdn_sequence_without_slot_has_no_state():
    _, mixer, builder = _gdn_setup(seed=31, slots=3)
    before = _cpu(mixer.ssm_state).clone()
    conv_before = _cpu(mixer.conv_state).clone()
    n = 2
    tables = (torch.zeros(n, 64, dtype=torch.int32, device=DEV),
              torch.zeros(n, 8, dtype=torch.int32, device=DEV))
    batch = builder.build([0, 4], [5, 3], [0] * 8, *tables, torch.arange(n, dtype=torch.int32),
                          [-1, 7])   # no slot, slot past the pool
    x = _bf16((8, 512), 32)
    got = mixer(x.to(DEV), batch)
    torch.cuda.synchronize()
    assert torch.equal(_cpu(mixer.ssm_state), before)
    assert torch.equal(_cpu(mixer.conv_state), conv_before)
    zeros_ssm = torch.zeros(2, 4, 128, 128)
    zeros_conv = torch.zeros(2, 3, mixer.conv_state.shape[2], dtype=torch.bfloat16)
    want = H.gdn_mixer(x, _gdn_params(mixer), zeros_conv, zeros_ssm,
                       [(list(range(5)), 0), (list(range(5, 8)), 1)], key_heads=2,
                       value_heads=4, key_dim=128, value_dim=128, eps=1e-6)
    _close(got.cpu(), want, "gdn without state")


@pytest.mark.parametrize("bound", [None, 1])
def test_gdn_recurrence_length_bound(bound):
    """Sequences of 16+ tokens run on the chunked kernel, unless the caller
    bounds every sequence below 16 tokens (a decode batch): then the per-token
    kernel takes them all. Either way each sequence's output and state follow
    the oracle's per-token rule, so a bound that is too small costs time only."""
    gen = torch.Generator().manual_seed(41)
    hk, hv, lens = 2, 4, [3, 40, 1, 17, 200]  # 200: three full 64-token chunks and a partial one
    tokens = sum(lens)
    q = torch.nn.functional.normalize(torch.randn(tokens, hk, 128, generator=gen), dim=-1) / 128 ** 0.5
    k = torch.nn.functional.normalize(torch.randn(tokens, hk, 128, generator=gen), dim=-1)
    v = torch.randn(tokens, hv, 128, generator=gen).to(torch.bfloat16)
    g = -0.5 * torch.rand(tokens, hv, generator=gen)
    beta = torch.rand(tokens, hv, generator=gen)
    state0 = 0.05 * torch.randn(5, hv, 128, 128, generator=gen)
    qsl = torch.tensor([0] + np.cumsum(lens).tolist(), dtype=torch.int32)
    slots = torch.tensor([2, 0, 3, 1, 4], dtype=torch.int64)
    state = state0.to(DEV)
    print(f"[hybrid] gdn recurrence, bound {bound}", flush=True)
    o = L.gdn_recurrence(q.to(DEV), k.to(DEV), v.to(DEV), g.to(DEV), beta.to(DEV), state,
                         qsl.to(DEV), slots.to(DEV), hk, hv, max_query_len=bound)
    torch.cuda.synchronize()
    kh = torch.arange(hv) // (hv // hk)  # value head h reads key head h / (hv / hk)
    for i, n in enumerate(lens):
        rows, slot = slice(int(qsl[i]), int(qsl[i]) + n), int(slots[i])
        want_o, want_s = H.gated_delta_rule(q[rows][:, kh], k[rows][:, kh], v[rows].float(),
                                            g[rows], beta[rows], state0[slot])
        _close(o[rows].cpu(), want_o, f"gdn recurrence output, sequence of {n}")
        _close(state[slot].cpu(), want_s, f"gdn recurrence state, sequence of {n}", 1e-2, 1e-3)


def test_decode_graph_replay_equals_eager():
    """The whole model's uniform decode step from a HIP graph equals eager, for
    a batch other than the captured one (new tokens and positions)."""
    wl = _workload(seed=7)
    start = [t.clone() for t in wl.layer_states()]

    def restore():
        for t, s0 in zip(wl.layer_states(), start):
            t.copy_(s0)

    graph = HybridDecodeGraph(wl.model, wl.build_decode())
    base = list(wl.computed)
    for trial in (1, 2):
        wl.computed[:4] = [c + trial for c in base[:4]]
        wl.token_ids[:4] = (wl.token_ids[:4] + 17 * trial) % CFG.vocab_size
        restore()
        eager = wl.model.forward(wl.build_decode()).clone()
        eager_states = [t.clone() for t in wl.layer_states()]
        restore()
        got = graph.replay(wl.build_decode()).clone()
        torch.cuda.synchronize()
        print(f"[hybrid] decode graph trial {trial}: max diff "
              f"{(got - eager).abs().max().item():.3e}", flush=True)
        assert torch.equal(got, eager)
        for a, b in zip(wl.layer_states(), eager_states):
            assert torch.equal(a, b)


def test_hybrid_serving_batch_properties(monkeypatch):
    """The full-size model (32 layers, hidden 4096, 8 QSA layers at 16q/2kv,
    top-k 2048) on the serving batch: 112 decode requests at 4k-32k context
    and 16 prefill chunks of 512 tokens."""
    wl = make_serving_hybrid_workload(DEV, seed=11)
    cfg = wl.cfg
    batch = wl.build()
    index_queries = _record_index_queries(monkeypatch)
    logits = wl.model.forward(batch)
    torch.cuda.synchronize()
    print(f"[hybrid] serving batch: tokens={wl.num_tokens} logits {tuple(logits.shape)}",
          flush=True)
    assert torch.isfinite(logits).all()
    md = batch.qsa.compressed
    k = cfg.token_topk // cfg.compress_ratio
    qsa_layers = [layer for layer in wl.model.layers if layer.kind == "full_attention"]
    assert len(qsa_layers) == len(index_queries) == 8
    for layer in qsa_layers:
        logical_invariants(layer.mixer.layer.topk_indices_buffer[:wl.num_tokens],
                           md.logical_positions, md.seq_lens, md.token_to_req, md.visible_blocks,
                           cfg.compress_ratio, k)
    # top-k bit-exact on the last QSA layer for every decode row and 512
    # sampled prefill rows (the selection of most rows is active here)
    g = torch.Generator().manual_seed(5)
    nd = md.num_decode_tokens
    sample = torch.cat([torch.arange(nd),
                        nd + torch.randperm(wl.num_tokens - nd, generator=g)[:512]])
    last = qsa_layers[-1]
    _check_selection(len(wl.model.layers) - 1, last.mixer, batch, index_queries[-1], cfg,
                     rows_checked=sample)


def test_hybrid_serving_decode_graph_replay_equals_eager():
    """The full-size model's uniform decode step (112 requests) from a HIP
    graph equals eager launches, caches and states included."""
    wl = make_serving_hybrid_workload(DEV, seed=12)
    start = [t.clone() for t in wl.layer_states()]

    def restore():
        for t, s0 in zip(wl.layer_states(), start):
            t.copy_(s0)

    graph = HybridDecodeGraph(wl.model, wl.build_decode())
    n = graph.num_tokens
    base = list(wl.computed)
    wl.computed[:n] = [c + 1 for c in base[:n]]
    restore()
    eager = wl.model.forward(wl.build_decode()).clone()
    eager_states = [t.clone() for t in wl.layer_states()]
    restore()
    got = graph.replay(wl.build_decode()).clone()
    torch.cuda.synchronize()
    print(f"[hybrid] serving decode graph: requests={n} max diff "
          f"{(got - eager).abs().max().item():.3e}", flush=True)
    assert torch.isfinite(got).all()
    assert torch.equal(got, eager)
    for a, b in zip(wl.layer_states(), eager_states):
        assert torch.equal(a, b)



def test_recorded_gemm_choices_load_and_agree_with_library_default():
    """The committed TunableOp records load on this software stack, and every
    recorded solution computes what the library's default choice computes
    (bf16 GEMMs at the recorded serving shapes, fp32 accumulation in both)."""
    import torch.nn.functional as F

    from qsa_vllm_amd.gemm_tuning import TUNING_FILE, disable_tuned_gemms, enable_tuned_gemms

    shapes = []
    for line in TUNING_FILE.read_text().splitlines():
        op, params = line.split(",")[:2]
        if op.startswith("Validator"):
            continue
        # column-major BLAS view of F.linear: m = out features, n = tokens
        m, n, k = (int(v) for v in params.split("_")[1:4])
        shapes.append((m, n, k, op.startswith("GemmAndBias")))
    assert len(shapes) >= 10
    g = torch.Generator(device=DEV).manual_seed(3)
    cases = []
    for m, n, k, bias in shapes:
        x = torch.randn(n, k, device=DEV, dtype=torch.bfloat16, generator=g)
        w = (0.02 * torch.randn(m, k, device=DEV, generator=g)).to(torch.bfloat16)
        b = torch.randn(m, device=DEV, generator=g).to(torch.bfloat16) if bias else None
        cases.append((x, w, b))
    want = [F.linear(x, w, b) for x, w, b in cases]
    assert enable_tuned_gemms()
    try:
        got = [F.linear(x, w, b) for x, w, b in cases]
        torch.cuda.synchronize()
    finally:
        disable_tuned_gemms()
    for (m, n, k, _), a, b in zip(shapes, got, want):
        err = (a.float() - b.float()).abs().max().item()
        scale = b.float().abs().max().item()
        print(f"[hybrid] recorded GEMM {m}x{n}x{k}: max diff {err:.3e} of {scale:.3e}", flush=True)
        assert err <= 0.02 * scale
