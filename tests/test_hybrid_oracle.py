"""CPU pins of the hybrid decoder oracle (oracle/hybrid_oracle.py), and the
host-side checks of the hybrid layer ops (no GPU needed)."""

import math

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


# ------------------------------------------------------------------ pins of the layer statements

def test_bf16_rounds_to_nearest_even():
    x = torch.tensor([1 + 2 ** -8, 1 + 3 * 2 ** -8, -(1 + 2 ** -8), 3.0 + 2 ** -20],
                     dtype=torch.float64)
    got = H.bf16(x)
    assert got.dtype == torch.bfloat16
    # halfway cases go to the even mantissa; 3 + 2^-20 is below half an ulp of 3
    assert got.double().tolist() == [1.0, 1 + 2 ** -6, -1.0, 3.0]


def test_rms_norm_zero_row_is_zero():
    w = torch.ones(16, dtype=torch.bfloat16)
    assert torch.equal(H.rms_norm(torch.zeros(2, 16, dtype=torch.bfloat16), w, 1e-6),
                       torch.zeros(2, 16, dtype=torch.bfloat16))


def _bf(t):
    return t.to(torch.bfloat16)


def _norm_inputs(tokens, hidden, rank, seed):
    g = _gen(seed)
    x = _bf(torch.randn(tokens, hidden, generator=g))
    res = _bf(torch.randn(tokens, hidden, generator=g))
    w = _bf(1 + 0.2 * torch.randn(hidden, generator=g))
    down = _bf(torch.randn(rank, hidden, generator=g) * 0.3)
    up = _bf(torch.randn(hidden, rank, generator=g) * 0.3)
    bias = _bf(torch.randn(hidden, generator=g))
    return x, res, w, down, up, bias


@pytest.mark.parametrize("with_residual", [False, True])
def test_gated_norm_zero_gate_weights(with_residual):
    """``model.py:85-98``: with both gate projections zero the gate is
    sigmoid(bias) per column: ``bf16(n * bf16(sigmoid(bias)))``, n the RMSNorm
    of x (+ residual, which is returned as the new residual)."""
    x, res, w, down, up, bias = _norm_inputs(5, 32, 4, seed=41)
    gated, new_res = H.gated_norm(x, res if with_residual else None, w, torch.zeros_like(down),
                                  torch.zeros_like(up), bias, 1e-6)
    src = _bf(x.double() + res.double()) if with_residual else x
    n = H.rms_norm(src, w, 1e-6)
    want = _bf(n.double() * _bf(torch.sigmoid(bias.double())).double())
    assert torch.equal(gated, want)
    if with_residual:
        assert torch.equal(new_res, src)
    else:
        assert new_res is None


def test_gated_norm_rank_one_gate_scalar_loops():
    """A rank-1 gate (only gate_down row 0 and gate_up column 0 nonzero),
    stated per element with scalar loops: d = bf16(sum_i n_i gd_0i),
    u_c = bf16(gu_c0 bf16(silu(d)) + b_c), out_c = bf16(n_c bf16(sigmoid(u_c)))."""
    x, _, w, down, up, bias = _norm_inputs(3, 16, 4, seed=42)
    down[1:] = 0
    up[:, 1:] = 0
    gated, _ = H.gated_norm(x, None, w, down, up, bias, 1e-6)
    n = H.rms_norm(x, w, 1e-6).double().tolist()
    gd, gu, b = down.double().tolist(), up.double().tolist(), bias.double().tolist()

    def r(v):
        return float(_bf(torch.tensor(v, dtype=torch.float64)).double())

    for t in range(3):
        d = r(sum(n[t][i] * gd[0][i] for i in range(16)))
        s = r(d / (1 + math.exp(-d)))
        for c in range(16):
            u = r(gu[c][0] * s + b[c])
            want = r(n[t][c] * r(1 / (1 + math.exp(-u))))
            assert float(gated[t, c]) == want, (t, c)


def test_swiglu_scalar_loops():
    """``act = bf16(silu(x W_gate^T) * (x W_up^T))``, ``out = bf16(act W_down^T)``;
    gate_up stacks the gate rows first (vLLM's MergedColumnParallelLinear),
    each product rounded to bf16 as the model's tensors are."""
    g = _gen(43)
    hidden, inter, tokens = 8, 5, 3
    x = _bf(torch.randn(tokens, hidden, generator=g))
    gate_up = _bf(torch.randn(2 * inter, hidden, generator=g) * 0.5)
    down = _bf(torch.randn(hidden, inter, generator=g) * 0.5)
    got = H.swiglu(x, gate_up, down)
    X, GU, D = x.double().tolist(), gate_up.double().tolist(), down.double().tolist()

    def r(v):
        return float(_bf(torch.tensor(v, dtype=torch.float64)).double())

    for t in range(tokens):
        act = []
        for j in range(inter):
            gt = r(sum(X[t][i] * GU[j][i] for i in range(hidden)))
            up = r(sum(X[t][i] * GU[inter + j][i] for i in range(hidden)))
            act.append(r(gt / (1 + math.exp(-gt)) * up))
        for c in range(hidden):
            assert float(got[t, c]) == r(sum(act[j] * D[c][j] for j in range(inter))), (t, c)
    zero_gate = gate_up.clone()
    zero_gate[:inter] = 0
    assert (H.swiglu(x, zero_gate, down) == 0).all()     # silu(0) = 0


def test_qsa_projection_split_index_map():
    """``attention.py:216-230``: columns [q|gate interleaved per head (2D each:
    query half, then gate half) | k | v | index], element by element."""
    T, heads, kv, D, idx = 2, 3, 2, 4, 5
    q_size, kv_size = heads * 2 * D, kv * D
    qkv = torch.arange(T * (q_size + 2 * kv_size + idx), dtype=torch.float32).view(T, -1)
    query, gate, key, value, index = H.qsa_projection_split(qkv, heads, kv, D, idx)
    for t in range(T):
        for h in range(heads):
            for d in range(D):
                assert query[t, h, d] == qkv[t, h * 2 * D + d]
                assert gate[t, h, d] == qkv[t, h * 2 * D + D + d]
        for j in range(kv):
            for d in range(D):
                assert key[t, j, d] == qkv[t, q_size + j * D + d]
                assert value[t, j, d] == qkv[t, q_size + kv_size + j * D + d]
        for i in range(idx):
            assert index[t, i] == qkv[t, q_size + 2 * kv_size + i]


# GDN mixer (vLLM 0.30.0 ``QwenGatedDeltaNetAttention``): per key head the
# qkvz projection holds [q (dk) | k (dk) | v (r dv) | z (r dv)] and ba holds
# [b (r) | a (r)], r = value heads per key head; value head h reads key head
# h // r. The causal conv runs over the channels [q of all key heads | k | v].
HK, HV, DK, DV, CONV = 2, 4, 4, 3, 3
R_GDN = HV // HK


def _gdn_params(hidden, seed, b_scale=1.0):
    g = _gen(seed)
    C = 2 * HK * DK + HV * DV
    return {
        "in_proj_qkvz": _bf(torch.randn(HK * (2 * DK + 2 * R_GDN * DV), hidden, generator=g) * 0.5),
        "in_proj_ba": _bf(torch.randn(HK * 2 * R_GDN, hidden, generator=g) * 0.5 * b_scale),
        "conv_weight": _bf(torch.randn(C, CONV, generator=g) * 0.5),
        "A_log": torch.randn(HV, generator=g) * 0.3,
        "dt_bias": torch.randn(HV, generator=g) * 0.3,
        "norm_weight": _bf(1 + 0.2 * torch.randn(DV, generator=g)),
        "out_proj": _bf(torch.randn(hidden, HV * DV, generator=g) * 0.5),
    }


def _gdn_split(x, p):
    """Per token: q, k [HK, DK], v, z [HV, DV], b, a [HV] (bf16-rounded projections)."""
    T = x.shape[0]
    qkvz = _bf(x.double() @ p["in_proj_qkvz"].double().T).double().view(T, HK, -1)
    ba = _bf(x.double() @ p["in_proj_ba"].double().T).double().view(T, HK, -1)
    q, k = qkvz[..., :DK], qkvz[..., DK:2 * DK]
    v = qkvz[..., 2 * DK:2 * DK + R_GDN * DV].reshape(T, HV, DV)
    z = qkvz[..., 2 * DK + R_GDN * DV:].reshape(T, HV, DV)
    return q, k, v, z, ba[..., :R_GDN].reshape(T, HV), ba[..., R_GDN:].reshape(T, HV)


def _gdn_out(core, z, p, eps):
    c = core.double()
    y = c / torch.sqrt((c * c).mean(-1, keepdim=True) + eps)
    y = _bf(y * p["norm_weight"].double() * F.silu(z))
    return _bf(y.reshape(core.shape[0], -1).double() @ p["out_proj"].double().T)


def _run_gdn(x, p, sequences, slots=1):
    conv = torch.zeros(slots, CONV - 1, 2 * HK * DK + HV * DV, dtype=torch.float64)
    ssm = torch.zeros(slots, HV, DK, DV, dtype=torch.float64)
    out = H.gdn_mixer(x, p, conv, ssm, sequences, key_heads=HK, value_heads=HV, key_dim=DK,
                      value_dim=DV, eps=1e-6)
    return out, conv, ssm


def _l2(v):
    return v / torch.sqrt((v * v).sum(-1, keepdim=True) + 1e-6)


def test_gdn_mixer_one_token_from_zero_state():
    """From zero states one token gives conv = silu(w[:, K-1] x) channel-wise,
    S = beta k v^T, so o = beta (k.q) v per value head, with q, k l2-normalised
    (q also scaled by dk^-0.5), beta = sigmoid(b), then the gated RMSNorm with
    silu(z) and out_proj."""
    hidden = 6
    p = _gdn_params(hidden, seed=44)
    x = _bf(torch.randn(1, hidden, generator=_gen(45)))
    got, _, _ = _run_gdn(x, p, [([0], 0)])
    q, k, v, z, b, _ = _gdn_split(x, p)
    mixed = torch.cat((q.reshape(1, -1), k.reshape(1, -1), v.reshape(1, -1)), -1)[0]
    conv = _bf(F.silu(p["conv_weight"].double()[:, -1] * mixed)).double()
    qc = _l2(conv[:HK * DK].view(HK, DK)) * DK ** -0.5
    kc = _l2(conv[HK * DK:2 * HK * DK].view(HK, DK))
    vc = conv[2 * HK * DK:].view(HV, DV)
    core = torch.zeros(1, HV, DV, dtype=torch.float64)
    for h in range(HV):
        j = h // R_GDN
        core[0, h] = torch.sigmoid(b[0, h]) * (kc[j] @ qc[j]) * vc[h]
    want = _gdn_out(_bf(core), z[:1], p, 1e-6)
    assert torch.equal(got, want)


def test_gdn_mixer_decay_without_write():
    """Token 2 with beta = 0 (b = -1000) writes nothing: its output is the
    decayed state of token 1 read by its own query,
    o2 = e^{g2} beta1 (k1.q2) v1, g = -exp(A_log) softplus(a + dt_bias)."""
    hidden = 6
    p = _gdn_params(hidden, seed=46)
    x = torch.zeros(2, hidden, dtype=torch.bfloat16)
    x[0, :5] = _bf(torch.randn(5, generator=_gen(47)))
    x[1, :5] = _bf(torch.randn(5, generator=_gen(48)))
    x[1, 5] = 1.0
    ba = p["in_proj_ba"].clone().view(HK, 2 * R_GDN, hidden)
    ba[:, :R_GDN, 5] = -1000.0                 # b of token 2 only (token 1 has x[5] = 0)
    p["in_proj_ba"] = ba.view(-1, hidden)
    got, _, _ = _run_gdn(x, p, [([0, 1], 0)])
    q, k, v, z, b, a = _gdn_split(x, p)
    mixed = torch.cat((q.reshape(2, -1), k.reshape(2, -1), v.reshape(2, -1)), -1)
    w = p["conv_weight"].double()
    conv = torch.stack([F.silu(w[:, -1] * mixed[0]),
                        F.silu(w[:, -2] * mixed[0] + w[:, -1] * mixed[1])])
    conv = _bf(conv).double()
    qc = _l2(conv[:, :HK * DK].view(2, HK, DK)) * DK ** -0.5
    kc = _l2(conv[:, HK * DK:2 * HK * DK].view(2, HK, DK))
    vc = conv[:, 2 * HK * DK:].view(2, HV, DV)
    gate = -torch.exp(p["A_log"].double()) * F.softplus(a[1] + p["dt_bias"].double())
    assert (torch.sigmoid(b[1]) == 0).all()
    core = torch.zeros(2, HV, DV, dtype=torch.float64)
    for h in range(HV):
        j = h // R_GDN
        beta1 = torch.sigmoid(b[0, h])
        core[0, h] = beta1 * (kc[0, j] @ qc[0, j]) * vc[0, h]
        core[1, h] = torch.exp(gate[h]) * beta1 * (kc[0, j] @ qc[1, j]) * vc[0, h]
    want = _gdn_out(_bf(core), z, p, 1e-6)
    assert torch.equal(got, want)


def test_gdn_mixer_state_hand_off():
    """A sequence processed in one call equals the same tokens in two calls
    with the conv and recurrent states carried between them; two sequences in
    one call keep their states apart."""
    hidden = 6
    p = _gdn_params(hidden, seed=49)
    x = _bf(torch.randn(7, hidden, generator=_gen(50)))
    whole, conv1, ssm1 = _run_gdn(x, p, [(list(range(5)), 0)])
    conv = torch.zeros(1, CONV - 1, 2 * HK * DK + HV * DV, dtype=torch.float64)
    ssm = torch.zeros(1, HV, DK, DV, dtype=torch.float64)
    kw = dict(key_heads=HK, value_heads=HV, key_dim=DK, value_dim=DV, eps=1e-6)
    first = H.gdn_mixer(x[:3], p, conv, ssm, [([0, 1, 2], 0)], **kw)
    second = H.gdn_mixer(x[3:5], p, conv, ssm, [([0, 1], 0)], **kw)
    assert torch.equal(torch.cat((first, second)), whole[:5])
    # float64 states agree to rounding (the projections' BLAS blocking depends on the row count)
    assert torch.equal(conv, conv1) and torch.allclose(ssm, ssm1, rtol=0, atol=1e-12)
    both, _, _ = _run_gdn(x, p, [(list(range(5)), 0), ([5, 6], 1)], slots=2)
    alone, _, _ = _run_gdn(x[5:7], p, [([0, 1], 0)])
    assert torch.equal(both[:5], whole[:5]) and torch.equal(both[5:], alone)
