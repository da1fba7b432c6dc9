"""CPU restatement of the hybrid decoder's layers around the QSA path.

TEST INFRASTRUCTURE ONLY: the reference that ``qsa_vllm_amd.hybrid`` and its
layer kernels (``qsa_vllm_amd.ops.hybrid_layers``) are tested against. Nothing under
``qsa_vllm_amd`` imports it.

Follows ``model.py:60-98`` (gated norm), ``:180-225`` (decoder layer),
``attention.py:145-234`` (QSA projection split, output gate, ``o_proj``) and
vLLM 0.30.0's ``QwenGatedDeltaNetAttention`` with its fla kernels
(``vllm/model_executor/layers/mamba/gdn/qwen_gdn_linear_attn.py``, not vendored
with the plugin): the published gated delta rule (Yang, Kautz, Hatamizadeh,
"Gated Delta Networks", ICLR 2025) in its per-token recurrent form, evaluated
in float64, one sequence at a time. Values are rounded to bf16 where the
model's tensors are bf16 (projection outputs, conv output, core output, norm
outputs); the arithmetic between those points is float64.

Pinning (``tests/test_hybrid_oracle.py``; ``tests/test_oracle_mutants.py``
plants a mistake in each function and requires its pin to fail): the
recurrence against an independent transition-matrix statement ``S_t = e^{g_t}
(I - beta_t k_t k_t^T) S_{t-1} + beta_t k_t v_t^T`` and closed forms (no
writes: pure decay; orthonormal keys: exact key-value recall and overwrite);
the convolution against ``torch.nn.functional.conv1d``; ``rms_norm`` against
closed forms (constant rows, power-of-two scaling, zero rows); ``gated_norm``
with zero gate weights (``n * bf16(sigmoid(bias))``) and a rank-1 gate stated
per element with scalar loops; ``swiglu`` by scalar loops (gate rows first)
and a zero gate; ``gdn_mixer`` by closed forms (one token from zero states:
``o = sigmoid(b) (k.q) v``; a second token with ``beta = 0``:
``o = e^g sigmoid(b1) (k1.q2) v1`` with ``g = -exp(A_log) softplus(a +
dt_bias)``) and the state hand-off (two calls equal one);
``qsa_projection_split`` against an explicit element index map.

Parity unpinned: vLLM's own GDN kernels (fla Triton, not vendored) - no golden
vectors of theirs exist in the plugin.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

__all__ = ["bf16", "rms_norm", "gated_norm", "swiglu", "causal_conv", "gated_delta_rule",
           "gdn_mixer", "qsa_projection_split"]


def bf16(x):
    return x.to(torch.bfloat16)


def rms_norm(x, weight, eps):
    """vLLM RMSNorm on bf16 rows: ``bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w)``."""
    xf = x.double()
    inv = 1.0 / torch.sqrt((xf * xf).mean(-1, keepdim=True) + eps)
    return bf16(bf16(xf * inv).double() * weight.double())


def gated_norm(x, residual, weight, gate_down, gate_up, gate_up_bias, eps):
    """``YuLanGatedNorm`` (model.py:85-98). Returns (gated, residual)."""
    if residual is not None:
        x = bf16(x.double() + residual.double())
        residual = x
    n = rms_norm(x, weight, eps)
    down = bf16(n.double() @ gate_down.double().T)
    up = bf16(bf16(F.silu(down.double())).double() @ gate_up.double().T + gate_up_bias.double())
    gated = bf16(n.double() * bf16(torch.sigmoid(up.double())).double())
    return gated, residual


def swiglu(x, gate_up, down):
    i = down.shape[1]
    gu = bf16(x.double() @ gate_up.double().T)
    act = bf16(F.silu(gu[:, :i].double()) * gu[:, i:].double())
    return bf16(act.double() @ down.double().T)


def causal_conv(x, weight, state):
    """One sequence: ``x`` [L, C], ``weight`` [C, K], ``state`` [K-1, C] (the
    previous K-1 inputs, oldest first). Returns (silu(conv) [L, C] float64,
    new state [K-1, C])."""
    K = weight.shape[1]
    padded = torch.cat((state.double(), x.double()), 0)
    L = x.shape[0]
    out = torch.zeros(L, x.shape[1], dtype=torch.float64)
    for t in range(L):
        for j in range(K):
            out[t] += weight[:, j].double() * padded[t + j]
    return F.silu(out), padded[L:L + K - 1].clone()


def gated_delta_rule(q, k, v, g, beta, state):
    """One sequence, per head: ``q, k`` [L, H, dk] (already normalised),
    ``v`` [L, H, dv], ``g, beta`` [L, H], ``state`` [H, dk, dv]. Per token:
    ``S <- e^g S``; ``u = beta (v - S^T k)``; ``S <- S + k u^T``; ``o = S^T q``.
    Returns (o [L, H, dv], state), float64."""
    S = state.double().clone()
    L, H = q.shape[:2]
    out = torch.zeros(L, H, v.shape[-1], dtype=torch.float64)
    for t in range(L):
        for h in range(H):
            S[h] *= torch.exp(g[t, h].double())
            kt = k[t, h].double()
            u = beta[t, h].double() * (v[t, h].double() - kt @ S[h])
            S[h] += torch.outer(kt, u)
            out[t, h] = q[t, h].double() @ S[h]
    return out, S


def gdn_mixer(x, p, conv_state, ssm_state, sequences, *, key_heads, value_heads, key_dim,
              value_dim, eps):
    """The GDN mixer on bf16 rows ``x`` [T, hidden]. ``p``: in_proj_qkvz,
    in_proj_ba, conv_weight [C, K], A_log, dt_bias, norm_weight, out_proj.
    ``sequences``: (token rows in order, state slot) per sequence. Updates the
    states in place; returns bf16 [T, hidden]."""
    T = x.shape[0]
    hk, hv, dk, dv = key_heads, value_heads, key_dim, value_dim
    r = hv // hk
    qkvz = bf16(x.double() @ p["in_proj_qkvz"].double().T).view(T, hk, 2 * dk + 2 * r * dv)
    ba = bf16(x.double() @ p["in_proj_ba"].double().T).view(T, hk, 2 * r)
    q, k = qkvz[..., :dk], qkvz[..., dk:2 * dk]
    v = qkvz[..., 2 * dk:2 * dk + r * dv].reshape(T, hv, dv)
    z = qkvz[..., 2 * dk + r * dv:].reshape(T, hv, dv)
    b, a = ba[..., :r].reshape(T, hv), ba[..., r:].reshape(T, hv)
    mixed = torch.cat((q.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1)), -1)
    g = -torch.exp(p["A_log"].double()) * F.softplus(a.double() + p["dt_bias"].double())
    beta = torch.sigmoid(b.double())
    core = torch.zeros(T, hv, dv, dtype=torch.bfloat16)
    for rows, slot in sequences:
        rows = torch.as_tensor(rows, dtype=torch.int64)
        conv, conv_state[slot] = causal_conv(mixed[rows], p["conv_weight"], conv_state[slot])
        conv = bf16(conv).double()
        L = rows.numel()
        qs = conv[:, :hk * dk].view(L, hk, dk)
        ks = conv[:, hk * dk:2 * hk * dk].view(L, hk, dk)
        vs = conv[:, 2 * hk * dk:].view(L, hv, dv)
        qs = qs / torch.sqrt((qs * qs).sum(-1, keepdim=True) + 1e-6) * dk ** -0.5
        ks = ks / torch.sqrt((ks * ks).sum(-1, keepdim=True) + 1e-6)
        qs, ks = qs.repeat_interleave(r, 1), ks.repeat_interleave(r, 1)
        o, S = gated_delta_rule(qs, ks, vs, g[rows], beta[rows], ssm_state[slot])
        ssm_state[slot] = S.to(ssm_state.dtype)
        core[rows] = bf16(o)
    c = core.double()
    y = c / torch.sqrt((c * c).mean(-1, keepdim=True) + eps)
    y = bf16(y * p["norm_weight"].double() * F.silu(z.double()))
    return bf16(y.reshape(T, -1).double() @ p["out_proj"].double().T)


def qsa_projection_split(qkv, heads, kv_heads, head_dim, index_size):
    """``attention.py:216-230``: (query, gate, key, value, index_qk) of the
    fused projection; the query half of each head's 2*head_dim rows, then the gate."""
    T = qkv.shape[0]
    q_size, kv_size = heads * head_dim * 2, kv_heads * head_dim
    q, k, v, idx = qkv.split((q_size, kv_size, kv_size, index_size), -1)
    qg = q.reshape(T, heads, 2 * head_dim)
    return (qg[..., :head_dim], qg[..., head_dim:], k.reshape(T, kv_heads, head_dim),
            v.reshape(T, kv_heads, head_dim), idx)
