"""Stand-ins for the reference's query objects (the fields its context builder reads:
src/nano_inference/core/request.py:11-19, :31-35; kv_cache/block.py:11-14), and their
translation to the oracle's FullQuery."""
from __future__ import annotations

import enum
from types import SimpleNamespace
from typing import List, Optional

import torch

from oracle import metadata as meta


class Stage(enum.Enum):
    PREFILL = "prefill"
    RECOMPUTE = "recompute"
    DECODE = "decode"


def query(prompt: List[int], outputs: List[int], stage: Stage, block_ids: List[int],
          block_size: int, mrope: Optional[torch.Tensor] = None, rid: str = "q",
          images=None, grids=None):
    gi = SimpleNamespace(prompt_token_ids=list(prompt), mrope_position_ids=mrope,
                         images=images, image_grid_thw=grids)
    return SimpleNamespace(request_id=rid, generation_inputs=gi, output_token_ids=list(outputs),
                           stage=stage, kv_cache_block=SimpleNamespace(block_ids=list(block_ids),
                                                                       block_size=block_size))


def to_oracle(q) -> meta.FullQuery:
    return meta.FullQuery(q.generation_inputs.prompt_token_ids, q.output_token_ids,
                          q.stage.value, q.kv_cache_block.block_ids, q.kv_cache_block.block_size,
                          q.generation_inputs.mrope_position_ids, q.request_id)


def random_batch(seed: int, batch: int, block_size: int = 16, mrope: bool = False,
                 stages=(Stage.PREFILL, Stage.RECOMPUTE, Stage.DECODE), max_prompt: int = 300,
                 pool: int = 4096, short_tables: bool = False):
    """Seeded mixed batch; tables are slices of one permutation of the pool.  With
    ``short_tables`` some tables lack the block of the last position (the builder
    then uses the table's last block, as the reference does)."""
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(pool, generator=g).tolist()
    out, off = [], 0
    for i in range(batch):
        st = stages[int(torch.randint(0, len(stages), (1,), generator=g))]
        if mrope and i % 2 == 1 and st == Stage.PREFILL:
            st = Stage.DECODE  # a text prefill cannot join an mRoPE batch
        plen = int(torch.randint(1, max_prompt + 1, (1,), generator=g))
        nout = int(torch.randint(1 if st == Stage.DECODE else 0, 40, (1,), generator=g))
        prompt = torch.randint(0, 151936, (plen,), generator=g).tolist()
        outs = torch.randint(0, 151936, (nout,), generator=g).tolist()
        total = plen + nout
        nb = -(-total // block_size)
        if short_tables and i % 3 == 0 and nb > 1:
            nb -= 1
        blocks = perm[off:off + nb]
        off += nb
        mr = None
        if mrope and i % 2 == 0:
            base = torch.arange(plen, dtype=torch.int64)
            mr = torch.stack([base, base // 3, base % 7 + 100])
        out.append(query(prompt, outs, st, blocks, block_size, mr, rid=f"r{i}"))
    return out
