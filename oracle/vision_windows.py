"""Restatement of the ViT window permutation and chunk boundaries (oracle).

TEST INFRASTRUCTURE ONLY.

Follows src/nano_inference/layers/vision.py:365-412 (_get_window_index: pad the
merge-group grid with a -100 sentinel to a multiple of the window size, reshape
into windows, drop sentinels, cumulative counts times the merge unit,
unique_consecutive) and :443-453 (full-attention cu_seqlens, one chunk per frame).
"""
from __future__ import annotations

from typing import List, Tuple

import torch
import torch.nn.functional as F


def get_window_index(grid_thw: List[Tuple[int, int, int]], spatial_merge_size: int = 2,
                     window_size: int = 112, patch_size: int = 14):
    ws = window_size // spatial_merge_size // patch_size                    # :320
    unit = spatial_merge_size * spatial_merge_size
    window_index, cu = [], [0]
    offset = 0
    for t, h, w in grid_thw:
        lh, lw = h // spatial_merge_size, w // spatial_merge_size
        index = torch.arange(t * lh * lw).reshape(t, lh, lw)
        ph, pw = (ws - lh % ws) % ws, (ws - lw % ws) % ws
        nwh, nww = (lh + ph) // ws, (lw + pw) // ws
        padded = F.pad(index.float(), (0, pw, 0, ph), value=-100).long()
        padded = padded.reshape(t, nwh, ws, nww, ws).permute(0, 1, 3, 2, 4)
        padded = padded.reshape(t * nwh * nww, ws, ws)
        seqlens = (padded != -100).sum(dim=[1, 2])
        flat = padded.reshape(-1)
        window_index.append(flat[flat != -100] + offset)
        cu.extend((seqlens.cumsum(0) * unit + cu[-1]).tolist())
        offset += t * lh * lw
    wi = torch.cat(window_index)
    cws = torch.unique_consecutive(torch.tensor(cu, dtype=torch.int32))
    return wi, cws


def full_cu_seqlens(grid_thw: List[Tuple[int, int, int]]) -> torch.Tensor:
    gt = torch.tensor([t for t, _, _ in grid_thw], dtype=torch.int32)
    ghw = torch.tensor([h * w for _, h, w in grid_thw], dtype=torch.int32)
    cu = torch.repeat_interleave(ghw, gt).cumsum(0, dtype=torch.int32)
    return F.pad(cu, (1, 0), value=0)
