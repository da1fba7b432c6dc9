"""CPU pins of the hybrid decoder oracle (oracle/hybrid_oracle.py), and the
host-side checks of the hybrid layer ops (no GPU needed)."""

import pytest
import torch
import torch.nn.functional as F

from oracle import hybrid as H
from qsa_vllm_amd.hybrid import HybridBatchBuilder, HybridConfig
from qsa_vllm_amd.ops import hybrid_layers


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


def test_layer_ops_reject_host_tensors():
    x = torch.zeros(4, 512, dtype=torch.bfloat16)
    w = torch.ones(512, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        hybrid_layers.gated_norm(x, None, w, torch.zeros(16, 512, dtype=torch.bfloat16),
                                 torch.zeros(512, 16, dtype=torch.bfloat16), w, 1e-6)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        hybrid_layers.silu_mul(torch.zeros(4, 64, dtype=torch.bfloat16))


def test_batch_builder_rows_and_sequences():
    cfg = HybridConfig(num_layers=4, hidden_size=512, tp_size=1, vocab_size=64)
    builder = HybridBatchBuilder(cfg, max_requests=4, max_tokens=40, main_table_width=8,
                                 comp_table_width=2, device="cpu")
    tables = torch.zeros(4, 8, dtype=torch.int32), torch.zeros(4, 2, dtype=torch.int32)
    b = builder.build([40, 3, 0, 21], [1, 1, 19, 9], list(range(30)), *tables,
                      torch.arange(4, dtype=torch.int32), [5, 1, 0, 3])
    assert b.num_tokens == 30 and b.num_decode_tokens == 2
    assert b.logits_rows.tolist() == [0, 1, 20, 29]
    assert b.query_start_loc.tolist() == [0, 1, 2, 21, 30]
    assert b.token_to_seq.tolist() == [0, 1] + [2] * 19 + [3] * 9
    assert b.state_slots.tolist() == [5, 1, 0, 3]
