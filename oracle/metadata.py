"""Restatement of the context builder's attention metadata (oracle).

TEST INFRASTRUCTURE ONLY.

Follows src/nano_inference/engine/context_builder.py:83-193: per query, the
step's tokens (prompt for PREFILL, prompt + outputs for RECOMPUTE, the last
output for DECODE), start position = total length - step length,
context_lens = start + step length, a bool mask with [:len] True, block tables
zero-padded to the longest table (int32), and slots
block_ids[pos // BS] * BS + pos % BS with -1 padding (int64).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List

import torch

PREFILL, RECOMPUTE, DECODE = "prefill", "recompute", "decode"


@dataclass
class Query:
    prompt_len: int
    output_len: int
    stage: str
    block_ids: List[int]
    block_size: int


def build(queries: List[Query]):
    """Returns dict(context_lens, kv_block_tables, slot_mapping, attention_mask,
    position_ids, is_prefill) with the reference's dtypes."""
    is_prefill = any(q.stage in (PREFILL, RECOMPUTE) for q in queries)      # :87-91
    steps = []
    for q in queries:                                                       # :96-108
        if q.stage == PREFILL:
            steps.append(q.prompt_len)
        elif q.stage == RECOMPUTE:
            steps.append(q.prompt_len + q.output_len)
        else:
            steps.append(1)
    b, smax = len(queries), max(steps)
    position_ids = torch.zeros((b, smax), dtype=torch.long)
    context_lens = torch.zeros(b, dtype=torch.long)
    for i, (q, n) in enumerate(zip(queries, steps)):                        # :123-139
        start = q.prompt_len + q.output_len - n
        position_ids[i, :n] = torch.arange(start, start + n)
        context_lens[i] = start + n
    max_total = int(context_lens.max())                                     # :141-149
    attention_mask = torch.zeros((b, max_total), dtype=torch.bool)
    for i, n in enumerate(context_lens.tolist()):
        attention_mask[i, :n] = True
    max_blocks = max(len(q.block_ids) for q in queries)                     # :151-168
    block_tables = torch.zeros((b, max_blocks), dtype=torch.int32)
    slot_mapping = torch.full((b, smax), -1, dtype=torch.long)
    for i, q in enumerate(queries):
        block_tables[i, :len(q.block_ids)] = torch.tensor(q.block_ids, dtype=torch.int32)
        start = int(position_ids[i, 0])
        for j in range(steps[i]):                                           # :170-193
            pos = start + j
            bi = pos // q.block_size
            phys = q.block_ids[bi] if bi < len(q.block_ids) else q.block_ids[-1]
            slot_mapping[i, j] = phys * q.block_size + pos % q.block_size
    return dict(context_lens=context_lens, kv_block_tables=block_tables,
                slot_mapping=slot_mapping, attention_mask=attention_mask,
                position_ids=position_ids, is_prefill=is_prefill)
