"""Op-for-op PyTorch-CPU restatement of QK-RMSNorm and RoPE / mRoPE (oracle).

TEST INFRASTRUCTURE ONLY: imported by tests, never by the product.

These are the steps between the projections and the KV-cache write of the
reference's paged attention layer (src/nano_inference/layers/attention.py:254-265):
q_norm / k_norm (layers/norm.py:35-47), then the rotary module (layers/rotary.py:
8-33 and :89-130 for 1-D RoPE, :148-210 for the Qwen2.5-VL mRoPE).  The torch
ops and their order are the reference's, so the rounding points in a low
precision dtype (the fp32 norm cast back before the weight, cos/sin cast to the
activation dtype, each product and the sum rounded) are the reference's too.
"""
from __future__ import annotations

from typing import Optional, Sequence, Tuple

import torch


def inv_freq(head_dim: int, base: float) -> torch.Tensor:
    """1 / base^(2i / D), i < D/2, float32 (layers/rotary.py:99-103, :165-168)."""
    return 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """layers/norm.py:35-47: fp32 mean of squares, rsqrt, cast back, times weight."""
    xf = x.float()
    variance = xf.pow(2).mean(dim=-1, keepdim=True)
    xn = xf * torch.rsqrt(variance + eps)
    return xn.to(x.dtype) * weight


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """[x1, x2] -> [-x2, x1] over the last dim (layers/rotary.py:8-17)."""
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def _apply(q, k, cos, sin):
    """layers/rotary.py:19-33."""
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


def rope(q: torch.Tensor, k: torch.Tensor, position_ids: torch.Tensor,
         freqs_table: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """1-D RoPE (layers/rotary.py:105-130); q/k (B, S, H, D), position_ids (B, S)."""
    freqs = position_ids.float().unsqueeze(-1) * freqs_table.unsqueeze(0).unsqueeze(0)
    emb = torch.cat((freqs, freqs), dim=-1)
    cos = emb.cos().to(dtype=q.dtype).unsqueeze(2)
    sin = emb.sin().to(dtype=q.dtype).unsqueeze(2)
    return _apply(q, k, cos, sin)


def mrope(q: torch.Tensor, k: torch.Tensor, position_ids: torch.Tensor,
          freqs_table: torch.Tensor, section: Sequence[int]) -> Tuple[torch.Tensor, torch.Tensor]:
    """Qwen2.5-VL mRoPE (layers/rotary.py:184-210); position_ids (3, B, S).

    ``section`` is (n_t, n_h, n_w) in frequencies, summing to D/2 (rotary.py:160-163
    asserts that; a violation raises ValueError here).
    """
    n0, n1, n2 = (int(s) for s in section)
    if n0 + n1 + n2 != freqs_table.numel():
        raise ValueError(f"mrope section {tuple(section)} must sum to {freqs_table.numel()}")
    freqs = torch.cat([
        position_ids[0].float().unsqueeze(-1) * freqs_table[:n0],
        position_ids[1].float().unsqueeze(-1) * freqs_table[n0:n0 + n1],
        position_ids[2].float().unsqueeze(-1) * freqs_table[n0 + n1:],
    ], dim=-1)
    emb = torch.cat([freqs, freqs], dim=-1)
    cos = emb.cos().to(q.dtype).unsqueeze(2)
    sin = emb.sin().to(q.dtype).unsqueeze(2)
    return _apply(q, k, cos, sin)


def qk_norm_rope(q: torch.Tensor, k: torch.Tensor, q_weight: Optional[torch.Tensor],
                 k_weight: Optional[torch.Tensor], eps: float, position_ids: torch.Tensor,
                 freqs_table: torch.Tensor, section: Optional[Sequence[int]] = None
                 ) -> Tuple[torch.Tensor, torch.Tensor]:
    """attention.py:259-265: optional q_norm / k_norm, then RoPE (or mRoPE)."""
    if q_weight is not None:
        q = rms_norm(q, q_weight, eps)
    if k_weight is not None:
        k = rms_norm(k, k_weight, eps)
    if section is None:
        return rope(q, k, position_ids, freqs_table)
    return mrope(q, k, position_ids, freqs_table, section)
