"""Non-attention pieces that the attention modules own as submodules.

The reference attention layers construct an RMSNorm for QK-norm and a rotary
embedding (src/nano_inference/layers/attention.py:138-140, :356-360); a drop-in
replacement must own submodules with the same names, parameters and formulas
so that checkpoints load and outputs match.  These run as PyTorch ops on the
GPU (they are not part of the attention kernels).
"""
from __future__ import annotations

from typing import Tuple

import torch
import torch.nn as nn


class RMSNorm(nn.Module):
    """x * rsqrt(mean(x^2) + eps), computed in fp32, cast back, times weight.

    Same formula and cast points as src/nano_inference/layers/norm.py:35-47.
    """

    def __init__(self, hidden_size: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + self.eps)
        return xf.to(x.dtype) * self.weight


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """[x1, x2] -> [-x2, x1] over the last dim (src/nano_inference/layers/rotary.py:8-17)."""
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def _inv_freq(head_dim: int, base: float) -> torch.Tensor:
    return 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))


class RotaryEmbedding(nn.Module):
    """1-D RoPE, same tables and cast points as src/nano_inference/layers/rotary.py:60-130."""

    def __init__(self, head_dim: int, base: float = 10000.0):
        super().__init__()
        if head_dim % 2 != 0:
            raise ValueError(f"head_dim must be even for rotary embedding, got {head_dim}")
        self.head_dim = head_dim
        self.base = base
        self.register_buffer("inv_freq", _inv_freq(head_dim, base), persistent=False)

    def forward(self, q: torch.Tensor, k: torch.Tensor,
                position_ids: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        freqs = position_ids.float().unsqueeze(-1) * self.inv_freq
        emb = torch.cat((freqs, freqs), dim=-1)
        cos = emb.cos().to(dtype=q.dtype, device=q.device).unsqueeze(2)
        sin = emb.sin().to(dtype=q.dtype, device=q.device).unsqueeze(2)
        return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


class MRotaryEmbedding(nn.Module):
    """3-axis (temporal, height, width) RoPE of the Qwen2.5-VL decoder.

    Same section split and tables as src/nano_inference/layers/rotary.py:133-210;
    text tokens (equal axes) reduce to RotaryEmbedding.
    """

    def __init__(self, head_dim: int, base: float = 10000.0,
                 mrope_section: Tuple[int, int, int] = (16, 24, 24)):
        super().__init__()
        n0, n1, n2 = mrope_section
        if n0 + n1 + n2 != head_dim // 2:
            raise ValueError(f"mrope_section {mrope_section} must sum to head_dim//2")
        self.head_dim = head_dim
        self.base = base
        self._section_freqs = (n0, n1, n2)
        self.register_buffer("inv_freq", _inv_freq(head_dim, base), persistent=False)

    def forward(self, q: torch.Tensor, k: torch.Tensor,
                position_ids: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        n0, n1, _ = self._section_freqs
        f = self.inv_freq
        freqs = torch.cat(
            [position_ids[0].float().unsqueeze(-1) * f[:n0],
             position_ids[1].float().unsqueeze(-1) * f[n0:n0 + n1],
             position_ids[2].float().unsqueeze(-1) * f[n0 + n1:]],
            dim=-1,
        )
        emb = torch.cat([freqs, freqs], dim=-1)
        cos = emb.cos().to(q.dtype).unsqueeze(2)
        sin = emb.sin().to(q.dtype).unsqueeze(2)
        return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin
