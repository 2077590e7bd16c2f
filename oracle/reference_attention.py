"""Op-for-op PyTorch-CPU restatement of the reference attention path (oracle).

TEST INFRASTRUCTURE ONLY: imported by tests, smoke() and bench.py's
cpu_baseline leg, never by the product.

Each function follows the cited lines of the reference (paths relative to the
reference repository) with the same torch ops in the same order, so that its
numerics (dtype of scores, fp32 softmax cast back to the input dtype) and its
cost profile (per-token write loop with .item(), padded gather,
repeat_interleave, materialised scores) are the reference's.
"""
from __future__ import annotations

import math
from typing import Optional

import torch


def sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
         attention_mask: Optional[torch.Tensor] = None, is_causal: bool = True) -> torch.Tensor:
    """src/nano_inference/layers/attention.py:12-50."""
    d = q.shape[-1]
    sq, sk = q.shape[-2], k.shape[-2]
    scores = torch.matmul(q, k.transpose(-2, -1)) / math.sqrt(d)           # :27
    if is_causal and sq == sk:                                              # :33-38
        tri = torch.triu(torch.ones(sq, sk, dtype=torch.bool, device=q.device), diagonal=1)
        scores = scores.masked_fill(tri, float("-inf"))
    if attention_mask is not None:                                          # :40-47
        if attention_mask.shape[-1] > sk:
            attention_mask = attention_mask[..., :sk]
        scores = scores + attention_mask.to(device=scores.device, dtype=scores.dtype)
    w = torch.softmax(scores.float(), dim=-1).to(q.dtype)                   # :49
    return torch.matmul(w, v)                                               # :50


def additive_mask(mask2d: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """bool (B, S) -> additive (B, 1, 1, S) of 0 / -inf (attention.py:321-326)."""
    add = torch.zeros_like(mask2d, dtype=dtype).masked_fill(~mask2d, float("-inf"))
    return add.view(mask2d.shape[0], 1, 1, -1)


def kv_write_loop(k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """src/nano_inference/layers/attention.py:267-278 (one layer's cache, in place).

    k, v: (B, S_step, H_kv, D); slot_mapping: (B, S_step) int64.
    """
    bs = k_cache.shape[2]
    for b in range(k.shape[0]):
        for s in range(k.shape[1]):
            slot = slot_mapping[b, s].item()
            if slot < 0:
                continue
            k_cache[slot // bs, :, slot % bs, :] = k[b, s]
            v_cache[slot // bs, :, slot % bs, :] = v[b, s]


def paged_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    k_cache: torch.Tensor, v_cache: torch.Tensor,
                    slot_mapping: torch.Tensor, block_tables: torch.Tensor,
                    context_lens: torch.Tensor, attention_mask: Optional[torch.Tensor],
                    is_prefill: bool) -> torch.Tensor:
    """Steps 3-8 of PagedCausalSelfAttention.forward (attention.py:267-332).

    q: (B, S, H, D) after QK-norm and RoPE; k, v: (B, S, H_kv, D); caches are one
    layer's [NB, H_kv, BS, D]; attention_mask: bool (B, S_total) or None.
    Returns the attention output (B, S, H, D) before o_proj.
    """
    b, s, h, d = q.shape
    hkv = k.shape[2]
    kv_write_loop(k, v, k_cache, v_cache, slot_mapping)                     # :267-278
    if is_prefill:                                                          # :281-284
        kc, vc = k, v
    else:                                                                   # :285-305
        max_ctx = context_lens.max().item()
        bs = k_cache.shape[2]
        tok = torch.arange(max_ctx).unsqueeze(0).expand(b, -1)
        phys = torch.gather(block_tables.long(), 1, tok // bs)
        kc = k_cache[phys, :, tok % bs, :]
        vc = v_cache[phys, :, tok % bs, :]
    if hkv != h:                                                            # :310-314
        kc = kc.repeat_interleave(h // hkv, dim=2)
        vc = vc.repeat_interleave(h // hkv, dim=2)
    qt, kt, vt = q.transpose(1, 2), kc.transpose(1, 2), vc.transpose(1, 2)  # :316-319
    mask = None
    if attention_mask is not None and attention_mask.dim() == 2:            # :321-326
        mask = additive_mask(attention_mask, q.dtype)
    out = sdpa(qt, kt, vt, attention_mask=mask, is_causal=True)             # :330-332
    return out.transpose(1, 2)


def decode_context_mask(context_lens: torch.Tensor) -> torch.Tensor:
    """Bool (B, max_len) with [:len] True (context_builder.py:141-149)."""
    max_len = int(context_lens.max().item())
    ar = torch.arange(max_len).unsqueeze(0)
    return ar < context_lens.unsqueeze(1)


def vision_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     cu_seqlens: torch.Tensor) -> torch.Tensor:
    """Per-chunk non-causal attention of src/nano_inference/layers/vision.py:190-208.

    q, k, v: (S, H, D) after RoPE.  Returns (S, H*D) before proj.
    """
    lengths = (cu_seqlens[1:] - cu_seqlens[:-1]).tolist()                   # :191
    parts = []
    for qc, kc, vc in zip(q.split(lengths, 0), k.split(lengths, 0), v.split(lengths, 0)):
        qc = qc.transpose(0, 1).unsqueeze(0)                                # :199-201
        kc = kc.transpose(0, 1).unsqueeze(0)
        vc = vc.transpose(0, 1).unsqueeze(0)
        a = sdpa(qc, kc, vc, is_causal=False)                               # :202
        parts.append(a.squeeze(0).transpose(0, 1).reshape(-1, q.shape[1] * q.shape[2]))
    return torch.cat(parts, dim=0)
