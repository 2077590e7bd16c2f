"""Drop-in context builder: the step's model inputs and attention metadata built on
the GPU from one upload.

``GenerateContextBuilder(device).build(queries)`` returns the same tensors as the
reference's builder (src/nano_inference/engine/context_builder.py:83-242): padded
``input_ids`` / ``position_ids`` / ``attention_mask``, ``AttentionMetadata`` with
``context_lens`` (int64), ``kv_block_tables`` (int32, zero-padded) and
``slot_mapping`` (int64, -1 padding), the mRoPE positions of VLM batches, token
histories and the prefill images.  The reference fills them with per-query
``torch.tensor`` calls and per-token ``.item()`` loops; here the host packs one
int64 descriptor per step (headers, token ids, block ids, explicit mRoPE rows),
copies it to the device once, and ``nia_step_metadata`` expands it in one launch.

The context also carries ``last_token_index`` (step length - 1 per row), so the
next-token logits can be read at each sequence's true last token
(``select_last_logits``); the reference reads column ``step_len - 1`` of the padded
step for every row (src/nano_inference/inferencer/torch_inferencer.py:242-251),
which is a padding column for the shorter prompts of a mixed-length prefill batch.

Queries are read by duck typing, as the reference's ``GenerateQuery``:
``stage`` (an enum whose value is "prefill", "recompute" or "decode", or that
string), ``generation_inputs.prompt_token_ids`` / ``mrope_position_ids`` /
``images`` / ``image_grid_thw``, ``output_token_ids``, ``request_id`` and
``kv_cache_block.block_ids`` / ``block_size``.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, List, Optional, Sequence

import numpy as np
import torch

from . import _lib
from .context import AttentionMetadata, GenerateContext

HEADER_WORDS = 8

_PREFILL, _RECOMPUTE, _DECODE = "prefill", "recompute", "decode"


def _stage(q) -> str:
    s = getattr(q.stage, "value", q.stage)
    s = str(s).lower()
    if s not in (_PREFILL, _RECOMPUTE, _DECODE):
        raise ValueError(f"query {getattr(q, 'request_id', '?')}: stage {s!r} has no step")
    return s


def _as_int64(x) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        return x.detach().to("cpu", torch.int64).numpy()
    return np.asarray(x, dtype=np.int64)


@dataclass
class PackedStep:
    """Host side of one step: the descriptor and the output sizes."""

    desc: np.ndarray  # int64: headers, tokens, blocks, mRoPE rows
    num_tokens: int
    num_blocks: int
    num_mrope: int
    batch: int
    max_step: int
    max_total: int
    max_blocks: int
    block_size: int
    has_mrope: bool
    is_prefill: bool


def pack_queries(queries: Sequence[Any]) -> PackedStep:
    """The step descriptor of ``queries`` (host only; no device work).

    Header of sequence i: step_len, start_pos, num_blocks, token_offset,
    block_offset, mrope_explicit e, mrope_offset, mrope_base c (positions of the
    mRoPE rows are the e explicit entries, then c, c + 1, ...).
    """
    if not queries:
        raise ValueError("Cannot build context for empty queries list.")
    b = len(queries)
    stages = [_stage(q) for q in queries]
    steps: List[np.ndarray] = []
    for q, st in zip(queries, stages):
        prompt = q.generation_inputs.prompt_token_ids
        if st == _PREFILL:
            steps.append(_as_int64(prompt))
        elif st == _RECOMPUTE:
            steps.append(np.concatenate([_as_int64(prompt), _as_int64(q.output_token_ids)]))
        else:
            if not q.output_token_ids:
                raise ValueError(f"decode query {q.request_id} has no output token")
            steps.append(_as_int64(q.output_token_ids[-1:]))
    blocks = [_as_int64(q.kv_cache_block.block_ids) for q in queries]
    has_mrope = any(q.generation_inputs.mrope_position_ids is not None for q in queries)

    hdr = np.zeros((b, HEADER_WORDS), dtype=np.int64)
    mrope_rows: List[np.ndarray] = []
    tok_off = blk_off = mr_off = 0
    for i, (q, st, s, bl) in enumerate(zip(queries, stages, steps, blocks)):
        n = len(s)
        start = len(q.generation_inputs.prompt_token_ids) + len(q.output_token_ids) - n
        e, base = 0, start
        if has_mrope:
            qm = q.generation_inputs.mrope_position_ids
            plen = len(q.generation_inputs.prompt_token_ids)
            if st == _PREFILL:
                if qm is None:
                    raise ValueError(f"prefill query {q.request_id} in an mRoPE batch has no "
                                     "mrope_position_ids")
                e = n
            elif st == _RECOMPUTE and qm is not None:
                e = plen
            if qm is not None:
                qm = _as_int64(qm)
                if qm.ndim != 2 or qm.shape[0] != 3 or qm.shape[1] < max(e, 1):
                    raise ValueError(f"query {q.request_id}: mrope_position_ids must be "
                                     f"(3, >= {max(e, 1)})")
                if e:
                    mrope_rows.append(np.ascontiguousarray(qm[:, :e]).reshape(-1))
                if st == _RECOMPUTE:
                    base = int(qm[0, -1]) + 1
                elif st == _DECODE:
                    base = int(qm[0, -1]) + len(q.output_token_ids)
        hdr[i] = (n, start, len(bl), tok_off, blk_off, e, mr_off, base)
        tok_off += n
        blk_off += len(bl)
        mr_off += 3 * e
    parts = [hdr.reshape(-1)] + steps + blocks + mrope_rows
    desc = np.concatenate(parts) if len(parts) > 1 else parts[0]
    ctx = hdr[:, 0] + hdr[:, 1]
    return PackedStep(
        desc=desc, num_tokens=tok_off, num_blocks=blk_off, num_mrope=mr_off, batch=b,
        max_step=int(hdr[:, 0].max()), max_total=int(ctx.max()),
        max_blocks=int(max(len(x) for x in blocks)),
        block_size=int(queries[0].kv_cache_block.block_size), has_mrope=has_mrope,
        is_prefill=any(st in (_PREFILL, _RECOMPUTE) for st in stages))


class GenerateContextBuilder:
    """Same constructor and ``build`` as the reference's builder
    (src/nano_inference/engine/context_builder.py:8-16, :83); the tensors are made
    on ``device`` (a GPU) by one upload and one kernel launch."""

    def __init__(self, device: torch.device):
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("GenerateContextBuilder builds on the GPU; got device "
                             f"{self.device}")

    def build(self, queries: Sequence[Any]) -> GenerateContext:
        pk = pack_queries(queries)
        dev = self.device
        if dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        desc = torch.from_numpy(pk.desc).pin_memory().to(dev, non_blocking=True)
        b, s = pk.batch, pk.max_step
        i64 = dict(dtype=torch.int64, device=dev)
        input_ids = torch.empty((b, s), **i64)
        position_ids = torch.empty((b, s), **i64)
        slot_mapping = torch.empty((b, s), **i64)
        context_lens = torch.empty((b,), **i64)
        last_index = torch.empty((b,), **i64)
        mask = torch.empty((b, pk.max_total), dtype=torch.bool, device=dev)
        tables = torch.empty((b, pk.max_blocks), dtype=torch.int32, device=dev)
        mrope = torch.empty((3, b, s), **i64) if pk.has_mrope else None
        lib = _lib.load()
        with torch.cuda.device(dev):
            stream = torch.cuda.current_stream(dev).cuda_stream
        st = lib.nia_step_metadata(
            desc.data_ptr(), pk.num_tokens, pk.num_blocks, pk.num_mrope, b, s, pk.max_total,
            pk.max_blocks, pk.block_size, input_ids.data_ptr(), position_ids.data_ptr(),
            slot_mapping.data_ptr(), context_lens.data_ptr(), last_index.data_ptr(),
            mask.data_ptr(), tables.data_ptr(), mrope.data_ptr() if mrope is not None else None,
            stream)
        _lib.check("nia_step_metadata", st)
        metadata = AttentionMetadata(context_lens=context_lens, kv_block_tables=tables,
                                     slot_mapping=slot_mapping, is_prefill=pk.is_prefill,
                                     mrope_position_ids=mrope)
        histories = [list(q.generation_inputs.prompt_token_ids) + list(q.output_token_ids)
                     for q in queries]
        images = grids = None
        if pk.is_prefill:                       # context_builder.py:214-230
            all_images: List[Any] = []
            all_grids: List[Any] = []
            for q in queries:
                gi = q.generation_inputs
                if _stage(q) in (_PREFILL, _RECOMPUTE) and getattr(gi, "images", None):
                    all_images.extend(gi.images)
                    if getattr(gi, "image_grid_thw", None):
                        all_grids.extend(gi.image_grid_thw)
            if all_images:
                images, grids = all_images, (all_grids or None)
        return GenerateContext(input_ids=input_ids, attention_mask=mask,
                               position_ids=position_ids, metadata=metadata,
                               request_ids=[q.request_id for q in queries],
                               token_histories=histories, images=images, image_grid_thw=grids,
                               last_token_index=last_index)


def select_last_logits(logits: torch.Tensor, context: GenerateContext) -> torch.Tensor:
    """(B, S, V) step logits -> (B, V) at each row's last real token."""
    idx = context.last_token_index
    if idx is None:
        raise ValueError("context has no last_token_index")
    rows = torch.arange(logits.shape[0], device=logits.device)
    return logits[rows, idx.to(logits.device)]
