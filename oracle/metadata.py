"""Restatement of the context builder's attention metadata (oracle).

TEST INFRASTRUCTURE ONLY.

Follows src/nano_inference/engine/context_builder.py:83-193: per query, the
step's tokens (prompt for PREFILL, prompt + outputs for RECOMPUTE, the last
output for DECODE), start position = total length - step length,
context_lens = start + step length, a bool mask with [:len] True, block tables
zero-padded to the longest table (int32), and slots
block_ids[pos // BS] * BS + pos % BS with -1 padding (int64).  build_context()
adds the padded input_ids and the mRoPE positions (:18-81).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional

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


@dataclass
class FullQuery:
    """A query with its token ids and optional mRoPE table (the fields of the
    reference's GenerateQuery that the context builder reads)."""
    prompt_token_ids: List[int]
    output_token_ids: List[int]
    stage: str
    block_ids: List[int]
    block_size: int
    mrope_position_ids: Optional[torch.Tensor] = None  # (3, prompt_len) int64
    request_id: str = ""


def build_context(queries: List[FullQuery]):
    """build() plus input_ids and the mRoPE positions, loop for loop as
    src/nano_inference/engine/context_builder.py:83-193 and :18-81 build them."""
    if not queries:
        raise ValueError("Cannot build context for empty queries list.")      # :84-85
    base = build([Query(len(q.prompt_token_ids), len(q.output_token_ids), q.stage, q.block_ids,
                        q.block_size) for q in queries])
    steps = []
    for q in queries:                                                       # :96-108
        if q.stage == PREFILL:
            steps.append(list(q.prompt_token_ids))
        elif q.stage == RECOMPUTE:
            steps.append(list(q.prompt_token_ids) + list(q.output_token_ids))
        else:
            steps.append([q.output_token_ids[-1]])
    b, smax = len(queries), max(len(s) for s in steps)
    input_ids = torch.zeros((b, smax), dtype=torch.long)                    # :113-131
    for i, s in enumerate(steps):
        input_ids[i, :len(s)] = torch.tensor(s, dtype=torch.long)
    position_ids = base["position_ids"]
    mrope = None
    if any(q.mrope_position_ids is not None for q in queries):              # :28-33
        mrope = torch.zeros((3, b, smax), dtype=torch.long)
        for i, (q, s) in enumerate(zip(queries, steps)):
            n = len(s)
            qm = q.mrope_position_ids
            if q.stage == PREFILL:                                          # :44-47
                if qm is None:
                    raise ValueError("a prefill query in an mRoPE batch needs its positions")
                mrope[:, i, :n] = qm[:, :n]
            elif q.stage == RECOMPUTE:                                      # :49-66
                plen = len(q.prompt_token_ids)
                if qm is not None:
                    mrope[:, i, :plen] = qm[:, :plen]
                    last = int(qm[0, -1].item())
                    for j, _ in enumerate(q.output_token_ids):
                        for a in range(3):
                            mrope[a, i, plen + j] = last + j + 1
                else:
                    for j in range(n):
                        for a in range(3):
                            mrope[a, i, j] = int(position_ids[i, j].item())
            else:                                                           # :68-77
                if qm is not None:
                    pos = int(qm[0, -1].item()) + len(q.output_token_ids)
                else:
                    pos = int(position_ids[i, 0].item())
                for a in range(3):
                    mrope[a, i, 0] = pos
    base.update(input_ids=input_ids, mrope_position_ids=mrope,
                token_histories=[list(q.prompt_token_ids) + list(q.output_token_ids)
                                 for q in queries],
                request_ids=[q.request_id for q in queries])
    return base
