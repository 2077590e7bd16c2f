"""Vision-tower attention (Qwen2.5-VL ViT) on the gfx950 varlen kernel.

``VisionAttention`` mirrors ``Qwen25VLVisionAttention`` of
src/nano_inference/layers/vision.py:155-208: fused qkv projection, 2-D RoPE,
then non-causal attention inside each chunk of ``cu_seqlens`` (an image for the
full-attention blocks, a window for the others) and the output projection.  The
reference loops over chunks in Python with one sdpa call each and a host sync
(:190-206); here one kernel launch covers every chunk.  As in the reference the
effective softmax scale is 1/sqrt(head_dim) (the stored ``scale`` attribute is
never used there, :169).

``window_index`` and ``full_cu_seqlens`` produce the chunk boundaries the way
src/nano_inference/layers/vision.py:365-412 and :443-453 do.
"""
from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import numpy as np
import torch
import torch.nn as nn

from . import ops
from .layers import rotate_half


def apply_rotary_pos_emb_vision(q, k, cos, sin):
    """2-D RoPE on (S, H, D) tensors, cos/sin (S, D), cast to q's dtype first."""
    cos = cos.unsqueeze(1).to(q.dtype)
    sin = sin.unsqueeze(1).to(q.dtype)
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


class VisionAttentionBase(nn.Module):
    """Marker base, as src/nano_inference/layers/vision.py:50-63."""


class VisionAttention(VisionAttentionBase):
    """Bidirectional packed multi-head attention of the ViT, one launch per layer."""

    def __init__(self, hidden_size: int, num_heads: int):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = hidden_size // num_heads
        self.scale = self.head_dim ** -0.5
        self.qkv = nn.Linear(hidden_size, hidden_size * 3, bias=True)
        self.proj = nn.Linear(hidden_size, hidden_size)

    def forward(
        self,
        x: torch.Tensor,
        cu_seqlens: torch.Tensor,
        position_embeddings: Tuple[torch.Tensor, torch.Tensor],
        max_seqlen: Optional[int] = None,
    ) -> torch.Tensor:
        seq_len = x.shape[0]
        cos, sin = position_embeddings
        qkv = self.qkv(x).reshape(seq_len, 3, self.num_heads, self.head_dim)
        q, k, v = qkv.permute(1, 0, 2, 3).unbind(0)
        q, k = apply_rotary_pos_emb_vision(q, k, cos, sin)
        out = ops.varlen_attention(q, k, v, cu_seqlens, max_seqlen_q=max_seqlen, causal=False)
        return self.proj(out.reshape(seq_len, self.num_heads * self.head_dim))


def full_cu_seqlens(grid_thw: Sequence[Tuple[int, int, int]]) -> np.ndarray:
    """One chunk per image frame: cumulative sums of h*w repeated t times, led by 0."""
    lens = [h * w for t, h, w in grid_thw for _ in range(t)]
    return np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)


def window_index(
    grid_thw: Sequence[Tuple[int, int, int]],
    spatial_merge_size: int = 2,
    window_size: int = 112,
    patch_size: int = 14,
) -> Tuple[np.ndarray, np.ndarray]:
    """Window permutation of merge groups and cumulative window lengths.

    Each frame's (h/m) x (w/m) grid of merge groups (m = spatial_merge_size) is
    cut into ws x ws windows, ws = window_size // m // patch_size, row-major over
    windows and row-major inside each; windows clipped at the frame edge keep
    their valid groups, empty windows vanish.  Returns (permutation of group ids,
    int32 cumulative token counts with a leading 0, m*m tokens per group).
    """
    ws = window_size // spatial_merge_size // patch_size
    unit = spatial_merge_size * spatial_merge_size
    order: List[np.ndarray] = []
    bounds = [0]
    offset = 0
    for t, h, w in grid_thw:
        gh, gw = h // spatial_merge_size, w // spatial_merge_size
        ids = np.arange(t * gh * gw).reshape(t, gh, gw)
        for ti in range(t):
            for wy in range(0, gh, ws):
                for wx in range(0, gw, ws):
                    blk = ids[ti, wy:wy + ws, wx:wx + ws].reshape(-1)
                    if blk.size == 0:
                        continue
                    order.append(blk + offset)
                    bounds.append(bounds[-1] + blk.size * unit)
        offset += t * gh * gw
    perm = np.concatenate(order) if order else np.zeros(0, dtype=np.int64)
    return perm, np.asarray(bounds, dtype=np.int32)
