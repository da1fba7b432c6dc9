"""CPU pins of the hybrid decoder oracle (oracle/hybrid_oracle.py) and the
PyTorch GDN pieces (qsa_vllm_amd/gdn.py, the GDN mixer of qsa_vllm_amd/hybrid.py)
checked against it."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import hybrid as H
from qsa_vllm_amd import gdn
from qsa_vllm_amd.hybrid import GatedDeltaNet, HybridBatchBuilder, HybridConfig, _Init


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _unit(*shape, seed):
    x = torch.randn(*shape, generator=_gen(seed), dtype=torch.float64)
    return x / x.norm(dim=-1, keepdim=True)


def _inputs(L, heads, dk, dv, seed):
    g = _gen(seed)
    q = _unit(L, heads, dk, seed=seed + 1) * dk ** -0.5
    k = _unit(L, heads, dk, seed=seed + 2)
    v = torch.randn(L, heads, dv, generator=g, dtype=torch.float64)
    decay = -torch.rand(L, heads, generator=g, dtype=torch.float64)
    beta = torch.rand(L, heads, generator=g, dtype=torch.float64)
    s0 = torch.randn(heads, dk, dv, generator=g, dtype=torch.float64) * 0.3
    return q, k, v, decay, beta, s0


def test_recurrence_matches_transition_matrices():
    q, k, v, g, beta, s0 = _inputs(11, 3, 6, 5, seed=1)
    o, S = H.gated_delta_rule(q, k, v, g, beta, s0)
    eye = torch.eye(6, dtype=torch.float64)
    for h in range(3):
        s = s0[h].clone()
        for t in range(11):
            kt = k[t, h]
            s = torch.exp(g[t, h]) * (eye - beta[t, h] * torch.outer(kt, kt)) @ s \
                + beta[t, h] * torch.outer(kt, v[t, h])
            assert torch.allclose(o[t, h], s.T @ q[t, h], atol=1e-12)
        assert torch.allclose(S[h], s, atol=1e-12)


def test_no_writes_is_pure_decay():
    q, k, v, g, _, s0 = _inputs(7, 2, 4, 3, seed=2)
    o, S = H.gated_delta_rule(q, k, v, g, torch.zeros(7, 2, dtype=torch.float64), s0)
    G = g.cumsum(0)
    for t in range(7):
        for h in range(2):
            assert torch.allclose(o[t, h], torch.exp(G[t, h]) * (s0[h].T @ q[t, h]), atol=1e-12)
    assert torch.allclose(S, torch.exp(G[-1])[:, None, None] * s0, atol=1e-12)


def test_orthonormal_keys_recall_and_overwrite():
    # Undecayed full-strength writes under orthonormal keys store each value
    # exactly; writing a key again replaces its value (plain linear attention
    # would add the two).
    dk, dv = 4, 3
    eye = torch.eye(dk, dtype=torch.float64)
    keys = torch.stack([eye[0], eye[1], eye[2], eye[1]])[:, None, :]
    vals = torch.randn(4, 1, dv, generator=_gen(3), dtype=torch.float64)
    zeros = torch.zeros(4, 1, dtype=torch.float64)
    _, S = H.gated_delta_rule(keys, keys, vals, zeros, torch.ones(4, 1, dtype=torch.float64),
                              torch.zeros(1, dk, dv, dtype=torch.float64))
    for i, want in ((0, vals[0, 0]), (1, vals[3, 0]), (2, vals[2, 0])):
        assert torch.allclose(eye[i] @ S[0], want, atol=1e-12)
    assert torch.allclose(eye[3] @ S[0], torch.zeros(dv, dtype=torch.float64))


def test_causal_conv_matches_conv1d():
    L, C, K = 9, 5, 4
    g = _gen(4)
    x = torch.randn(L, C, generator=g, dtype=torch.float64)
    w = torch.randn(C, K, generator=g, dtype=torch.float64)
    state = torch.randn(K - 1, C, generator=g, dtype=torch.float64)
    out, new_state = H.causal_conv(x, w, state)
    full = torch.cat((state, x), 0).T[None]                        # [1, C, K-1+L]
    want = F.silu(F.conv1d(full, w[:, None, :], groups=C))[0].T    # valid positions: L
    assert torch.allclose(out, want, atol=1e-12)
    assert torch.equal(new_state, torch.cat((state, x), 0)[-(K - 1):])


def test_rms_norm_closed_forms():
    w = (1 + 0.25 * torch.randn(64, generator=_gen(5))).to(torch.bfloat16)
    for c in (0.75, -3.0, 40.0):
        x = torch.full((2, 64), c, dtype=torch.bfloat16)
        # mean square c^2: x * inv rounds to sign(c) in bf16 (eps is far below half an ulp)
        want = (torch.sign(torch.tensor(c)) * w.float()).to(torch.bfloat16)
        assert torch.equal(H.rms_norm(x, w, 1e-6)[0], want)
    x = torch.randn(3, 64, generator=_gen(6)).to(torch.bfloat16)
    scaled = (x.double() * 4).to(torch.bfloat16)                  # exact power-of-two scale
    assert torch.equal(H.rms_norm(x, w, 0.0), H.rms_norm(scaled, w, 0.0))


@pytest.mark.parametrize("lengths,chunk", [([64], 16), ([37, 5, 16], 16), ([3], 8)])
def test_chunked_product_matches_recurrence(lengths, chunk):
    heads, dk, dv = 2, 8, 6
    B = len(lengths)
    L = -(-max(lengths) // chunk) * chunk
    q = torch.zeros(B, heads, L, dk)
    k, v = torch.zeros_like(q), torch.zeros(B, heads, L, dv)
    g, beta = torch.zeros(B, heads, L), torch.zeros(B, heads, L)
    s0 = torch.zeros(B, heads, dk, dv)
    want_o, want_s = [], []
    for b, n in enumerate(lengths):
        qq, kk, vv, gg, bb, ss = _inputs(n, heads, dk, dv, seed=10 + b)
        q[b, :, :n], k[b, :, :n], v[b, :, :n] = (u.transpose(0, 1).float() for u in (qq, kk, vv))
        g[b, :, :n], beta[b, :, :n] = gg.T.float(), bb.T.float()
        s0[b] = ss.float()
        o, S = H.gated_delta_rule(qq, kk, vv, gg, bb, ss)
        want_o.append(o)
        want_s.append(S)
    o, S = gdn.gdn_chunked(q, k, v, g, beta, s0, chunk=chunk)
    for b, n in enumerate(lengths):
        assert torch.allclose(o[b, :, :n].transpose(0, 1).double(), want_o[b], atol=2e-5)
        assert torch.allclose(S[b].double(), want_s[b], atol=2e-5)


def test_decode_product_matches_one_recurrence_step():
    heads, dk, dv = 3, 8, 5
    q, k, v, g, beta, _ = _inputs(4, heads, dk, dv, seed=20)
    state = torch.randn(6, heads, dk, dv, generator=_gen(21)) * 0.3
    slots = torch.tensor([4, 0, 5, 2])
    want = [H.gated_delta_rule(q[i:i + 1], k[i:i + 1], v[i:i + 1], g[i:i + 1], beta[i:i + 1],
                               state[int(s)]) for i, s in enumerate(slots)]
    before = state.clone()
    o = gdn.gdn_decode(q.float(), k.float(), v.float(), g.float(), beta.float(), state, slots)
    for i, s in enumerate(slots.tolist()):
        assert torch.allclose(o[i].double(), want[i][0][0], atol=1e-5)
        assert torch.allclose(state[s].double(), want[i][1], atol=1e-5)
    for s in (1, 3):
        assert torch.equal(state[s], before[s])


def test_conv_product_matches_oracle():
    C, K = 12, 4
    g = _gen(30)
    w = torch.randn(C, K, generator=g).to(torch.bfloat16)
    state = torch.randn(5, K - 1, C, generator=g).to(torch.bfloat16)
    lengths, slots = [6, 1, 2], torch.tensor([3, 0, 4])
    rows = torch.randn(sum(lengths), C, generator=g).to(torch.bfloat16)
    width = 8
    gather = torch.full((3, width), -1, dtype=torch.int64)
    at = 0
    for i, n in enumerate(lengths):
        gather[i, :n] = torch.arange(at, at + n)
        at += n
    tail = torch.tensor(lengths)[:, None] + torch.arange(K - 1)[None, :]
    ref_state = state.clone()
    out = gdn.conv_prefill(rows, w, state, slots, gather, tail)
    at = 0
    for i, n in enumerate(lengths):
        s = int(slots[i])
        want, new = H.causal_conv(rows[at:at + n], w, ref_state[s])
        assert torch.equal(out[i, :n], H.bf16(want))
        assert torch.equal(state[s], H.bf16(new))
        at += n
    # one decode token per sequence on the states just written
    x = torch.randn(3, C, generator=g).to(torch.bfloat16)
    ref_state = state.clone()
    out = gdn.conv_decode(x, w, state, slots)
    for i, s in enumerate(slots.tolist()):
        want, new = H.causal_conv(x[i:i + 1], w, ref_state[s])
        assert torch.equal(out[i], H.bf16(want[0]))
        assert torch.equal(state[s], H.bf16(new))


def _small_cfg(**kw):
    base = dict(num_layers=1, hidden_size=64, tp_size=1, linear_num_key_heads=2,
                linear_num_value_heads=4, linear_key_head_dim=16, linear_value_head_dim=16,
                gdn_chunk=8, vocab_size=97)
    base.update(kw)
    return HybridConfig(**base)


def _mixer_params(m):
    return {"in_proj_qkvz": m.in_proj_qkvz, "in_proj_ba": m.in_proj_ba,
            "conv_weight": m.conv_weight, "A_log": m.A_log, "dt_bias": m.dt_bias,
            "norm_weight": m.norm_weight, "out_proj": m.out_proj}


def test_gdn_mixer_cpu_matches_oracle():
    cfg = _small_cfg()
    init = _Init("cpu", 7, 0.1)
    mixer = GatedDeltaNet(cfg, init, num_slots=6, state_std=0.1)
    mixer.norm_weight = (1 + 0.2 * torch.randn(16, generator=_gen(8))).to(torch.bfloat16)
    computed, scheduled = [40, 3, 0, 21], [1, 1, 19, 9]
    slots = np.array([5, 1, 0, 3])
    builder = HybridBatchBuilder(cfg, max_requests=4, max_tokens=32, main_table_width=8,
                                 comp_table_width=2, device="cpu")
    tables = torch.zeros(4, 8, dtype=torch.int32), torch.zeros(4, 2, dtype=torch.int32)
    batch = builder.build(computed, scheduled, np.zeros(30, dtype=np.int64), *tables,
                          torch.arange(4, dtype=torch.int32), slots)
    x = (torch.randn(30, 64, generator=_gen(9))).to(torch.bfloat16)
    conv0, ssm0 = mixer.conv_state.clone(), mixer.ssm_state.clone()
    got = mixer(x, batch)
    starts = np.concatenate(([0], np.cumsum(scheduled)[:-1]))
    seqs = [(list(range(s, s + n)), int(slot)) for s, n, slot in zip(starts, scheduled, slots)]
    want = H.gdn_mixer(x, _mixer_params(mixer), conv0, ssm0, seqs, key_heads=2, value_heads=4,
                       key_dim=16, value_dim=16, eps=cfg.rms_norm_eps)
    err = (got.double() - want.double()).abs()
    scale = want.double().abs().max()
    assert err.max() <= 0.02 * scale and err.mean() <= 2e-3 * scale, (err.max(), scale)
    assert torch.equal(mixer.conv_state, conv0)
    assert torch.allclose(mixer.ssm_state.double(), ssm0.double(), atol=1e-4)
