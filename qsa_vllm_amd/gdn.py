"""Gated DeltaNet (GDN) token mixer of the hybrid decoder, in PyTorch-ROCm.

The model's linear-attention layers (``model.py:205-212``) are vLLM's
``QwenGatedDeltaNetAttention`` (vllm 0.30.0,
``vllm/model_executor/layers/mamba/gdn/qwen_gdn_linear_attn.py``, not part of
the plugin). Per sequence, per value head ``h`` (key head ``h // r``,
``r = value_heads / key_heads``), token ``t``:

* ``x_t = silu(sum_j w[:, j] * m_{t-K+1+j})``: depthwise causal convolution of
  width ``K`` over the projected ``q|k|v`` rows, the last ``K-1`` rows of the
  previous step carried in the conv state;
* ``q_t = l2norm(q_t) / sqrt(dk)``, ``k_t = l2norm(k_t)``;
  ``beta_t = sigmoid(b_t)``, ``g_t = -exp(A_log) * softplus(a_t + dt_bias)``;
* the gated delta rule on the state ``S`` ``[dk, dv]`` (fp32):
  ``S <- exp(g_t) S``, ``u_t = beta_t (v_t - S^T k_t)``, ``S <- S + k_t u_t^T``,
  ``o_t = S^T q_t``;
* ``y_t = rmsnorm(o_t) * w_norm * silu(z_t)``.

Decode tokens advance their sequence's state by one step (``gdn_decode``).
Prefill chunks run the chunked (WY) form of the same recurrence
(``gdn_chunked``): within a chunk of ``C`` tokens with cumulative log decay
``G``, ``(I + A) U = beta V - beta e^G K S_0`` with
``A[t, s] = beta_t e^{G_t - G_s} k_t.k_s`` (``s < t``),
``O = e^G Q S_0 + (M o Q K^T) U`` with ``M[t, s] = e^{G_t - G_s}`` (``s <= t``),
``S_C = e^{G_C} S_0 + (e^{G_C - G} K)^T U`` (Yang, Kautz, Hatamizadeh, "Gated
Delta Networks", ICLR 2025). Ragged chunks are padded with tokens whose
``g = beta = 0`` and ``q = k = v = 0``: such a step leaves the state unchanged.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

__all__ = ["conv_decode", "conv_prefill", "gdn_decode", "gdn_chunked", "gated_rmsnorm",
           "gdn_gates", "l2norm"]


def l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """fp32 ``x / sqrt(sum(x^2) + eps)`` over the last dim."""
    x = x.float()
    return x * torch.rsqrt((x * x).sum(-1, keepdim=True) + eps)


def gdn_gates(a: torch.Tensor, b: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor):
    """fp32 (log decay g, write strength beta) from the projected a, b [tokens, heads]."""
    g = -A_log.float().exp() * F.softplus(a.float() + dt_bias.float())
    return g, torch.sigmoid(b.float())


def conv_decode(mixed: torch.Tensor, weight: torch.Tensor, conv_state: torch.Tensor,
                slots: torch.Tensor) -> torch.Tensor:
    """One token per sequence: ``mixed`` [n, C] bf16, ``weight`` [C, K],
    ``conv_state`` [slots, K-1, C] (the last K-1 inputs, oldest first).
    Returns silu(conv) in bf16 and advances the states in place."""
    window = torch.cat((conv_state[slots], mixed[:, None, :]), dim=1)    # [n, K, C]
    out = torch.einsum("nkc,ck->nc", window.float(), weight.float())
    conv_state[slots] = window[:, 1:]
    return F.silu(out).to(mixed.dtype)


def conv_prefill(mixed: torch.Tensor, weight: torch.Tensor, conv_state: torch.Tensor,
                 slots: torch.Tensor, gather: torch.Tensor, tail: torch.Tensor) -> torch.Tensor:
    """Chunks of several sequences. ``gather`` [S, L] holds each padded
    position's token row in ``mixed`` or -1; ``tail`` [S, K-1] the rows of the
    padded sequence (state rows first, then the chunk) that become the new
    state. Returns silu(conv) as [S, L, C] bf16 (pad positions undefined) and
    writes the states in place."""
    S, L = gather.shape
    K = weight.shape[1]
    C = mixed.shape[1]
    rows = torch.where(gather >= 0, gather, torch.zeros_like(gather))
    x = mixed[rows.reshape(-1)].view(S, L, C)
    x = torch.where((gather >= 0)[..., None], x, torch.zeros_like(x))
    padded = torch.cat((conv_state[slots], x), dim=1).float()               # [S, K-1+L, C]
    w = weight.float()
    out = padded[:, 0:L] * w[:, 0]
    for j in range(1, K):
        out = out + padded[:, j:j + L] * w[:, j]
    new_state = torch.gather(padded, 1, tail[..., None].expand(S, K - 1, C))
    conv_state[slots] = new_state.to(conv_state.dtype)
    return F.silu(out).to(mixed.dtype)


def gdn_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
               beta: torch.Tensor, state: torch.Tensor, slots: torch.Tensor) -> torch.Tensor:
    """One recurrence step per sequence. ``q, k`` [n, H, dk] and ``v`` [n, H, dv]
    fp32 (q, k normalised and expanded to the value heads), ``g, beta`` [n, H],
    ``state`` [slots, H, dk, dv] fp32 updated in place. Returns o [n, H, dv] fp32."""
    S = state[slots]
    S.mul_(g.exp()[..., None, None])
    kS = torch.matmul(k.unsqueeze(-2), S).squeeze(-2)
    u = (v - kS) * beta[..., None]
    S.add_(k.unsqueeze(-1) * u.unsqueeze(-2))
    o = torch.matmul(q.unsqueeze(-2), S).squeeze(-2)
    state[slots] = S
    return o


def gdn_chunked(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
                beta: torch.Tensor, initial: torch.Tensor, chunk: int = 64):
    """Chunked gated delta rule. ``q, k`` [B, H, L, dk], ``v`` [B, H, L, dv],
    ``g, beta`` [B, H, L] fp32, ``initial`` [B, H, dk, dv]; ``L`` a multiple of
    ``chunk``. Returns (o [B, H, L, dv], final state [B, H, dk, dv]), fp32."""
    B, H, L, dk = q.shape
    dv = v.shape[-1]
    N, C = L // chunk, chunk
    q = q.reshape(B, H, N, C, dk)
    k = k.reshape(B, H, N, C, dk)
    v = v.reshape(B, H, N, C, dv)
    g = g.reshape(B, H, N, C)
    beta = beta.reshape(B, H, N, C)
    G = g.cumsum(-1)
    diff = G[..., :, None] - G[..., None, :]                               # G_t - G_s
    lower = torch.ones(C, C, dtype=torch.bool, device=q.device).tril()
    strict = lower.clone()
    strict.fill_diagonal_(False)
    ninf = torch.tensor(float("-inf"), device=q.device)
    within = torch.where(lower, diff, ninf).exp()                          # s <= t
    A = (beta[..., :, None] * torch.where(strict, diff, ninf).exp()
         * torch.matmul(k, k.transpose(-1, -2)))
    eye = torch.eye(C, dtype=q.dtype, device=q.device)
    T = torch.linalg.solve_triangular(eye + A, eye.expand_as(A), upper=False,
                                      unitriangular=True)
    Wv = torch.matmul(T, beta[..., None] * v)
    Wk = torch.matmul(T, (beta * G.exp())[..., None] * k)
    P = torch.matmul(q, k.transpose(-1, -2)) * within
    qg = G.exp()[..., None] * q
    kg = (G[..., -1:] - G).exp()[..., None] * k
    last = G[..., -1].exp()
    out = torch.empty(B, H, N, C, dv, dtype=q.dtype, device=q.device)
    S = initial.to(q.dtype).clone()
    for n in range(N):
        U = Wv[:, :, n] - torch.matmul(Wk[:, :, n], S)
        out[:, :, n] = torch.matmul(qg[:, :, n], S) + torch.matmul(P[:, :, n], U)
        S = last[:, :, n, None, None] * S + torch.matmul(kg[:, :, n].transpose(-1, -2), U)
    return out.reshape(B, H, L, dv), S


def gated_rmsnorm(o: torch.Tensor, z: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``rmsnorm(o) * weight * silu(z)`` over the last dim in fp32, bf16 out."""
    x = o.float()
    x = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps)
    return (x * weight.float() * F.silu(z.float())).to(torch.bfloat16)
