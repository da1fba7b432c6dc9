"""The hybrid decoder's other layers on gfx950: gated RMSNorm, SwiGLU
activation and the Gated DeltaNet mixer's kernels (``csrc/hybrid.hip``).

Each function checks dtypes, devices and layouts (RuntimeError), allocates its
outputs and calls the C ABI on the current stream of the tensors' device.
There is no eager fallback: the HIP library must be present.
"""

from __future__ import annotations

import torch

from .. import _lib
from ._torch_ops import _dtype, _on_gpu, _ptr, _require, _stream, _vector

__all__ = ["gated_norm", "silu_mul", "gdn_prep", "gdn_conv_state", "gdn_recurrence",
           "gdn_gated_norm"]

HEAD_DIM = 128


def _rows2d(t, name, width=None):
    _dtype(t, torch.bfloat16, name)
    _require(t.dim() == 2 and (t.size(1) <= 1 or t.stride(1) == 1),
             f"{name} must be [rows, width] with unit column stride")
    if width is not None:
        _require(t.size(1) == width, f"{name} must have {width} columns, got {t.size(1)}")


def gated_norm(x, residual, weight, gate_down, gate_up, gate_up_bias, eps, *, out=None):
    """``YuLanGatedNorm`` (model.py:85-98). With ``residual``, it becomes
    ``bf16(x + residual)`` in place and is normalised; without, ``x`` is
    normalised and is the residual. Returns (gated, residual)."""
    dev = _on_gpu(x, residual, weight, gate_down, gate_up, gate_up_bias, out)
    rows, hidden = x.shape
    _rows2d(x, "x")
    if residual is not None:
        _rows2d(residual, "residual", hidden)
        _require(residual.size(0) == rows, "residual must have the rows of x")
    for t, name in ((weight, "weight"), (gate_up_bias, "gate_up_bias")):
        _dtype(t, torch.bfloat16, name)
        _require(t.shape == (hidden,) and t.is_contiguous(), f"{name} must be contiguous [hidden]")
    rank = gate_down.size(0)
    for t, name, shape in ((gate_down, "gate_down", (rank, hidden)),
                           (gate_up, "gate_up", (hidden, rank))):
        _dtype(t, torch.bfloat16, name)
        _require(tuple(t.shape) == shape and t.is_contiguous(), f"{name} must be contiguous {shape}")
    if out is None:
        out = torch.empty(rows, hidden, dtype=torch.bfloat16, device=dev)
    _rows2d(out, "out", hidden)
    res_stride = residual.stride(0) if residual is not None else 0
    lib = _lib.load()
    nbytes = lib.qsa_gated_norm_workspace_bytes(rows, hidden)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev) if nbytes else None
    with torch.cuda.device(dev):
        _lib.call("qsa_gated_norm", _ptr(x), x.stride(0), _ptr(residual), res_stride,
                  _ptr(residual), res_stride, _ptr(weight), _ptr(gate_down), _ptr(gate_up),
                  _ptr(gate_up_bias), _ptr(out), out.stride(0), rows, hidden, rank, float(eps),
                  _ptr(ws), nbytes, _stream(dev))
    return out, (residual if residual is not None else x)


def silu_mul(gate_up):
    """``SiluAndMul``: [rows, 2 I] -> bf16(silu(gate) * up) [rows, I]."""
    dev = _on_gpu(gate_up)
    _rows2d(gate_up, "gate_up")
    rows, width = gate_up.shape
    _require(width % 2 == 0, "gate_up width must be even")
    out = torch.empty(rows, width // 2, dtype=torch.bfloat16, device=dev)
    with torch.cuda.device(dev):
        _lib.call("qsa_silu_mul", _ptr(gate_up), gate_up.stride(0), _ptr(out), out.stride(0),
                  rows, width // 2, _stream(dev))
    return out


def _check_qkvz(qkvz, key_heads, value_heads):
    _rows2d(qkvz, "qkvz")
    _require(key_heads > 0 and value_heads % key_heads == 0,
             "value heads must be a multiple of key heads")
    r = value_heads // key_heads
    _require(qkvz.size(1) == key_heads * (2 + 2 * r) * HEAD_DIM,
             "qkvz must hold [q, k, v, z] per key head with 128-dim heads")
    return (2 * key_heads + value_heads) * HEAD_DIM


def _gdn_common(qkvz, conv_state, query_start_loc, slots, key_heads, value_heads, conv_kernel):
    channels = _check_qkvz(qkvz, key_heads, value_heads)
    if conv_state is not None:
        _dtype(conv_state, torch.bfloat16, "conv_state")
        _require(conv_state.dim() == 3 and conv_state.is_contiguous()
                 and tuple(conv_state.shape[1:]) == (conv_kernel - 1, channels),
                 "conv_state must be contiguous [slots, K-1, channels]")
    _vector(query_start_loc, torch.int32, "query_start_loc")
    _vector(slots, torch.int64, "slots", query_start_loc.numel() - 1)
    return channels


def gdn_prep(qkvz, ba, conv_weight, conv_state, query_start_loc, token_to_seq, slots, A_log,
             dt_bias, key_heads, value_heads):
    """Conv + SiLU, l2-normalised q (scaled) and k, v, and the gates of every
    token. Returns (q [T, Hk, 128] fp32, k, v [T, Hv, 128] bf16, g [T, Hv] fp32, beta)."""
    dev = _on_gpu(qkvz, ba, conv_weight, conv_state, query_start_loc, token_to_seq, slots,
                  A_log, dt_bias)
    K = conv_weight.size(1)
    channels = _gdn_common(qkvz, conv_state, query_start_loc, slots, key_heads, value_heads, K)
    tokens = qkvz.size(0)
    _rows2d(ba, "ba", 2 * value_heads)
    _require(ba.size(0) == tokens, "ba must have the rows of qkvz")
    _dtype(conv_weight, torch.bfloat16, "conv_weight")
    _require(conv_weight.shape == (channels, K) and conv_weight.is_contiguous(),
             "conv_weight must be contiguous [channels, K]")
    _vector(token_to_seq, torch.int32, "token_to_seq", tokens)
    for t, name in ((A_log, "A_log"), (dt_bias, "dt_bias")):
        _vector(t, torch.float32, name, value_heads)
    q = torch.empty(tokens, key_heads, HEAD_DIM, dtype=torch.float32, device=dev)
    k = torch.empty_like(q)
    v = torch.empty(tokens, value_heads, HEAD_DIM, dtype=torch.bfloat16, device=dev)
    g = torch.empty(tokens, value_heads, dtype=torch.float32, device=dev)
    beta = torch.empty_like(g)
    with torch.cuda.device(dev):
        _lib.call("qsa_gdn_prep", _ptr(qkvz), qkvz.stride(0), _ptr(ba), ba.stride(0),
                  _ptr(conv_weight), _ptr(conv_state), conv_state.size(0), _ptr(query_start_loc),
                  _ptr(token_to_seq), _ptr(slots), query_start_loc.numel() - 1, _ptr(A_log),
                  _ptr(dt_bias), key_heads, value_heads, HEAD_DIM, K, tokens, _ptr(q), _ptr(k),
                  _ptr(v), _ptr(g), _ptr(beta), _stream(dev))
    return q, k, v, g, beta


def gdn_conv_state(qkvz, conv_state, query_start_loc, slots, key_heads, value_heads):
    """Store each sequence's last K-1 inputs as its conv state (after ``gdn_prep``)."""
    dev = _on_gpu(qkvz, conv_state, query_start_loc, slots)
    K = conv_state.size(1) + 1
    _gdn_common(qkvz, conv_state, query_start_loc, slots, key_heads, value_heads, K)
    with torch.cuda.device(dev):
        _lib.call("qsa_gdn_conv_state", _ptr(qkvz), qkvz.stride(0), qkvz.size(0), _ptr(conv_state),
                  conv_state.size(0), _ptr(query_start_loc), _ptr(slots),
                  query_start_loc.numel() - 1, key_heads, value_heads, HEAD_DIM, K, _stream(dev))


def gdn_recurrence(q, k, v, g, beta, state, query_start_loc, slots, key_heads, value_heads,
                   max_query_len=None):
    """The gated delta rule over each sequence (state updated in place).
    Returns o [T, Hv, 128] bf16. ``max_query_len``: the longest sequence's
    token count when the caller knows it (a decode batch: 1); below 16 the
    chunked kernel is not launched."""
    dev = _on_gpu(q, k, v, g, beta, state, query_start_loc, slots)
    tokens = q.size(0)
    for t, name in ((q, "q"), (k, "k")):
        _dtype(t, torch.float32, name)
        _require(t.shape == (tokens, key_heads, HEAD_DIM) and t.is_contiguous(),
                 f"{name} must be contiguous [tokens, key_heads, 128]")
    _dtype(v, torch.bfloat16, "v")
    _require(v.shape == (tokens, value_heads, HEAD_DIM) and v.is_contiguous(),
             "v must be contiguous [tokens, value_heads, 128]")
    for t, name in ((g, "g"), (beta, "beta")):
        _dtype(t, torch.float32, name)
        _require(t.shape == (tokens, value_heads) and t.is_contiguous(),
                 f"{name} must be contiguous [tokens, value_heads]")
    _dtype(state, torch.float32, "state")
    _require(state.dim() == 4 and tuple(state.shape[1:]) == (value_heads, HEAD_DIM, HEAD_DIM)
             and state.is_contiguous(), "state must be contiguous [slots, value_heads, 128, 128]")
    _vector(query_start_loc, torch.int32, "query_start_loc")
    _vector(slots, torch.int64, "slots", query_start_loc.numel() - 1)
    o = torch.empty(tokens, value_heads, HEAD_DIM, dtype=torch.bfloat16, device=dev)
    with torch.cuda.device(dev):
        _lib.call("qsa_gdn_recurrence", _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), tokens,
                  _ptr(state), state.size(0), _ptr(query_start_loc), _ptr(slots),
                  query_start_loc.numel() - 1, key_heads, value_heads, HEAD_DIM,
                  -1 if max_query_len is None else int(max_query_len), _ptr(o), _stream(dev))
    return o


def gdn_gated_norm(o, qkvz, weight, eps, key_heads, value_heads):
    """``rmsnorm(o) * weight * silu(z)`` per (token, value head), bf16 [T, Hv, 128]."""
    dev = _on_gpu(o, qkvz, weight)
    tokens = o.size(0)
    _check_qkvz(qkvz, key_heads, value_heads)
    _require(qkvz.size(0) == tokens, "qkvz must have the rows of o")
    _dtype(o, torch.bfloat16, "o")
    _require(o.shape == (tokens, value_heads, HEAD_DIM) and o.is_contiguous(),
             "o must be contiguous [tokens, value_heads, 128]")
    _dtype(weight, torch.bfloat16, "weight")
    _require(weight.shape == (HEAD_DIM,) and weight.is_contiguous(), "weight must be [128]")
    y = torch.empty_like(o)
    with torch.cuda.device(dev):
        _lib.call("qsa_gdn_gated_norm", _ptr(o), _ptr(qkvz), qkvz.stride(0), _ptr(weight),
                  float(eps), tokens, key_heads, value_heads, HEAD_DIM, _ptr(y), _stream(dev))
    return y
