"""Indexer RMSNorm and partial RoPE (ops/normalization.py of the reference plugin).

``rotary_cache`` builds the bf16 [positions, rotary_dim] table (cos, then sin)
exactly as the reference does, in fp32 on the given device;
``IndexerRMSNorm`` holds the learned gamma and epsilon; ``indexer_norm_rope``
runs RMSNorm + partial RoPE on a [tokens, heads, dim] tensor through
``libqsa_hip.so``.
"""

from __future__ import annotations

from functools import cache

import torch
from torch import nn

from . import _torch_ops  # noqa: F401  (registers torch.ops.yulan_qsa_kernels)

__all__ = ["rotary_cache", "IndexerRMSNorm", "indexer_norm_rope"]


@cache
def rotary_cache(max_position, rotary_dim, theta, device):
    """[max_position, rotary_dim] bf16: cos of every (position, channel) phase,
    then sin; phase = position * theta^(-2c / rotary_dim), all in fp32
    (ops/normalization.py:17-23)."""
    even = torch.arange(0, rotary_dim, 2, dtype=torch.float32, device=device)
    frequencies = theta ** (-even / rotary_dim)
    positions = torch.arange(max_position, dtype=torch.float32, device=device)
    angles = torch.outer(positions, frequencies)
    return torch.cat((angles.cos(), angles.sin()), dim=-1).to(torch.bfloat16)


def _copy_weight_loader(param: torch.Tensor, loaded_weight: torch.Tensor) -> None:
    """Checkpoint loader of the gamma: copy a tensor of the same shape into
    the parameter (what vLLM's ``default_weight_loader`` does for it)."""
    if param.shape != loaded_weight.shape:
        raise ValueError(f"weight of shape {tuple(loaded_weight.shape)} does not fit a parameter "
                         f"of shape {tuple(param.shape)}")
    param.data.copy_(loaded_weight)


def _default_weight_loader():
    try:
        from vllm.model_executor.model_loader.weight_utils import default_weight_loader
    except ImportError:
        return _copy_weight_loader
    return default_weight_loader


class IndexerRMSNorm(nn.Module):
    """Gamma (bf16, ones at init) and epsilon of an indexer RMSNorm
    (ops/normalization.py:26-31). The gamma carries the checkpoint loader
    vLLM's model loader calls: vLLM's ``default_weight_loader`` when vLLM is
    installed, else a shape-checked copy."""

    def __init__(self, width, epsilon):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(width, dtype=torch.bfloat16))
        self.weight.weight_loader = _default_weight_loader()
        self.variance_epsilon = epsilon


def indexer_norm_rope(values, norm, positions, cos_sin, rotary_dim):
    """RMSNorm (fp32 statistics, bf16 result times bf16 gamma) then rotate-half
    RoPE on the first ``rotary_dim`` dims at each token's position
    (ops/normalization.py:33-83). Returns a new [tokens, heads, dim] bf16 tensor."""
    output = torch.empty(values.shape, device=values.device, dtype=torch.bfloat16)
    torch.ops.yulan_qsa_kernels.indexer_norm_rope(
        values, norm.weight, positions, cos_sin, float(norm.variance_epsilon), int(rotary_dim),
        output)
    return output
