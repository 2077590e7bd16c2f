"""Per-step attention metadata, field-for-field the reference's contract.

Mirrors ``AttentionMetadata`` of src/nano_inference/core/context.py:7-24 so that
the reference's context builder (src/nano_inference/engine/context_builder.py:
83-242) and inferencer (src/nano_inference/inferencer/torch_inferencer.py:
221-222) can fill it unchanged.  The kernels read ``context_lens``,
``kv_block_tables`` and ``slot_mapping`` directly, in the reference's dtypes.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, List, Optional, Tuple

import torch


@dataclass
class AttentionMetadata:
    """Metadata required for paged attention: the reference's fields in its order,
    plus the optional row scales of fp8 caches and an optional caller-owned decode
    workspace (default None)."""

    context_lens: torch.Tensor  # (B,) int64 - total sequence length per request
    kv_block_tables: torch.Tensor  # (B, max_blocks_per_seq) int32, zero-padded
    slot_mapping: torch.Tensor  # (B, S_step) int64, -1 for padding

    # Physical cache tensors [L, num_blocks, H_kv, block_size, D]
    k_cache: Optional[torch.Tensor] = None
    v_cache: Optional[torch.Tensor] = None

    # Forward mode
    is_prefill: bool = False

    # VLM only: (3, B, S_step) mRoPE position ids; None for text-only batches.
    mrope_position_ids: Optional[torch.Tensor] = None

    # fp8 caches only (not in the reference): per-row scales [L, num_blocks, H_kv,
    # block_size] float32 beside uint8 / float8_e4m3fn k_cache / v_cache.
    k_scale: Optional[torch.Tensor] = None
    v_scale: Optional[torch.Tensor] = None

    # Not in the reference: a caller-owned decode workspace (uint8, at least
    # ops.decode_workspace_bytes(...) for the step's sizes) for decode calls that are
    # captured in a HIP graph, so that the graph holds memory its owner controls; None
    # uses the per-stream workspace of ops.decode_workspace.
    decode_workspace: Optional[torch.Tensor] = None


@dataclass
class GenerateContext:
    """Batch-level inputs of one engine step (fields of the reference's
    src/nano_inference/core/context.py:28-51), plus ``last_token_index``: the
    column of each row's last real token in the padded step, where the step's
    next-token logits must be read."""

    input_ids: torch.Tensor  # (B, S_step) int64
    attention_mask: torch.Tensor  # (B, S_total) bool
    position_ids: torch.Tensor  # (B, S_step) int64
    metadata: AttentionMetadata
    request_ids: List[str]
    token_histories: List[List[int]]
    images: Optional[List[Any]] = None
    image_grid_thw: Optional[List[Tuple[int, int, int]]] = None
    last_token_index: Optional[torch.Tensor] = None  # (B,) int64


@dataclass
class PackedAttentionMetadata(AttentionMetadata):
    """A step whose tokens lie back to back in one row, (1, T): sequences
    0 .. num_decode - 1 feed one token each (rows 0 .. num_decode - 1) and decode;
    the others feed a prefill chunk of q_len[s] rows from row q_start[s], on top of
    the context_lens[s] - q_len[s] tokens already cached.  Lets one step mix prefill
    chunks and decodes; the reference's batches are all-prefill or all-decode
    (src/nano_inference/scheduler/scheduler.py:176-230)."""

    q_start: Optional[torch.Tensor] = None  # (B,) int32
    q_len: Optional[torch.Tensor] = None  # (B,) int32
    num_decode: int = 0
    max_q_len: int = 0
