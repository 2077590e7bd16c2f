"""Drop-in attention layers backed by the gfx950 kernels.

Same names, constructor arguments, parameter names and forward signatures as
the reference's src/nano_inference/layers/attention.py:

* ``scaled_dot_product_attention(q, k, v, attention_mask=None, is_causal=True)``
  (:12-50) - the free function, also used by the vision tower;
* ``PagedCausalSelfAttention`` (:206-340) with ``.layer_idx`` and
  ``forward(x, position_ids, attention_mask=None, metadata=None)``;
* ``Qwen25VLDecoderAttention`` (:343-371), the mRoPE variant.

Projections stay PyTorch ops, as in the reference.  QK-RMSNorm, RoPE / mRoPE and
the KV-cache write run as one fused kernel (head_dim 128; other head dims keep the
PyTorch norm and rotary ops and the plain write kernel), and the block-table
gather, GQA, masking and softmax attention run in the attention kernels.  A
``PackedAttentionMetadata`` step (decodes and prefill chunks in one packed row)
splits its rows between the decode and the chunked-prefill kernel.  Differences
from the reference, all where the reference has no defined behaviour of its own:
* a decode step (``is_prefill`` False) with more than one new token per
  sequence attends with a bottom-right causal mask (chunked prefill); the
  reference applies no causal mask when S_q != S_k
  (src/nano_inference/layers/attention.py:33-38);
* a query row whose every key is masked gives zeros (the reference's softmax gives
  NaN).
Masks: a prefix (right-padding) mask, which is what the context builder produces
(src/nano_inference/engine/context_builder.py:141-149), becomes per-sequence key
lengths; any other mask is added to the scaled scores as the reference adds it
(src/nano_inference/layers/attention.py:40-47) by nia_prefill_masked.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import ops
from .context import AttentionMetadata, PackedAttentionMetadata
from .layers import MRotaryEmbedding, RMSNorm, RotaryEmbedding


_PREFIX = ops.TensorMemo()


def _prefix_lengths(mask: torch.Tensor, batch: int, key_len: int,
                    device: torch.device) -> Optional[torch.Tensor]:
    """Visible-key counts (int32, on ``device``) of a prefix mask, or None when the mask
    is not one (the general additive path then takes it).

    Prefix masks come in the reference's two forms: 2-D bool (B, S_total) with True =
    visible, or additive (B, 1, 1, S_total) with 0 = visible and -inf = masked.
    Checking that the mask is a prefix reads it back to the host; the result is kept
    per mask tensor (ops.TensorMemo), so the layers of a step that share one mask pay
    for that once.  A mask on the CPU is checked there.
    """
    key = (batch, key_len, device)
    lens = _PREFIX.get(mask, key)
    if lens is not None:
        return None if isinstance(lens, bool) else lens
    lens = False
    if mask.dim() == 2 and mask.shape[0] in (1, batch):
        vis = mask[:, :key_len].to(torch.bool)
    elif (mask.dim() == 4 and mask.shape[0] in (1, batch) and mask.shape[1] == 1
          and mask.shape[2] == 1):
        m = mask[:, 0, 0, :key_len]
        vis = m == 0
        if not torch.all(vis | (m == float("-inf"))):
            vis = None  # finite non-zero values: not a pure visibility mask
    else:
        vis = None
    if vis is not None and vis.shape[-1] == key_len:
        if vis.shape[0] != batch:
            vis = vis.expand(batch, -1)
        n = vis.sum(dim=-1)
        ar = torch.arange(vis.shape[-1], device=vis.device)
        if torch.equal(vis, ar.unsqueeze(0) < n.unsqueeze(1)):
            lens = n.to(device=device, dtype=torch.int32)
    _PREFIX.put(mask, key, lens)
    return None if lens is False else lens


def _additive_mask(mask: torch.Tensor, b: int, h: int, sq: int, sk: int,
                   dtype: torch.dtype) -> torch.Tensor:
    """The mask the reference adds to the (B, H, S_q, S_k) scores (src/nano_inference/
    layers/attention.py:40-47): sliced to S_k and cast to the scores' dtype, as a 4-D
    tensor that broadcasts against (B, H, S_q, S_k).  A 2-D bool (B, S) mask is the
    layers' visibility form (:321-326): True visible, False -inf."""
    if mask.shape[-1] > sk:
        mask = mask[..., :sk]
    if mask.dim() == 2 and mask.dtype == torch.bool:
        add = torch.zeros(mask.shape, dtype=dtype, device=mask.device)
        add = add.masked_fill(~mask, float("-inf"))
        mask = add.view(mask.shape[0], 1, 1, -1)
    else:
        mask = mask.to(dtype)
    while mask.dim() < 4:
        mask = mask.unsqueeze(0)
    try:
        torch.broadcast_shapes(mask.shape, (b, h, sq, sk))
    except RuntimeError:
        raise ValueError(f"attention_mask of shape {tuple(mask.shape)} does not broadcast "
                         f"to the scores ({b}, {h}, {sq}, {sk})") from None
    if mask.shape[-1] != sk:
        mask = mask.expand(*mask.shape[:3], sk)
    return mask


_INDEX_CACHE: dict = {}


def _seq_index(b: int, q_step: int, q_len: int, k_step: int, k_len: int,
               device: torch.device):
    """(q_start, q_len, k_start, k_len) int32 tensors for b equal sequences, built once
    per shape and device (the kernels only read them)."""
    key = (b, q_step, q_len, k_step, k_len, device)
    t = _INDEX_CACHE.get(key)
    if t is None:
        ar = torch.arange(b, dtype=torch.int32)
        t = tuple(x.to(device) for x in (ar * q_step, torch.full((b,), q_len, dtype=torch.int32),
                                          ar * k_step, torch.full((b,), k_len, dtype=torch.int32)))
        if len(_INDEX_CACHE) >= 64:
            _INDEX_CACHE.clear()
        _INDEX_CACHE[key] = t
    return t


def _token_rows(x: torch.Tensor):
    """A (B, H, S, D) tensor as token rows without a copy: (view (rows, H, D), step) with
    token s of batch b at row b * step + s, or None when its strides do not allow it.
    Both the (B, H, S, D) layout and a transposed (B, S, H, D) one do."""
    bb, hh, ss, dd = x.shape
    sb, sh, st, sd = x.stride()
    if sd != 1 or bb == 0 or ss == 0:
        return None
    if ss == 1:
        st = sb if bb > 1 else dd  # the stride of a size-1 dimension is arbitrary
    if st <= 0 or (bb > 1 and sb % st):
        return None
    step = sb // st if bb > 1 else 0
    rows = (bb - 1) * step + ss
    return x.as_strided((rows, hh, dd), (st, sh, 1)), step


def scaled_dot_product_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    attention_mask: Optional[torch.Tensor] = None,
    is_causal: bool = True,
) -> torch.Tensor:
    """softmax(q k^T / sqrt(D) [+ causal] [+ mask]) v on the gfx950 kernel.

    Shapes as in src/nano_inference/layers/attention.py:12-50: q (B, H, S_q, D),
    k, v (B, H_kv, S_k, D) (H_kv may divide H), output (B, H, S_q, D).  As in the
    reference the causal mask is applied only when S_q == S_k; the padding mask
    is sliced to S_k.  q, k and v are read in place (their (B, H, S, D) strides become
    per-sequence row offsets), and the output is written in q's layout.
    """
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be (B, H, S, D)")
    b, h, sq, d = q.shape
    sk = k.shape[2]
    causal = ops.CAUSAL_TOP_LEFT if (is_causal and sq == sk) else ops.CAUSAL_NONE
    dev = q.device
    out = torch.empty_like(q)
    rq, rk, rv, ro = (_token_rows(t) for t in (q, k, v, out))
    if rq and rk and rv and ro and rk[1] == rv[1] and ro[1] == rq[1]:
        (q3, q_step), (k3, k_step), (v3, _), (o3, _) = rq, rk, rv, ro
    else:  # other layouts: token-major copies
        q3 = q.transpose(1, 2).reshape(b * sq, h, d)
        k3 = k.transpose(1, 2).reshape(b * sk, k.shape[1], d)
        v3 = v.transpose(1, 2).reshape(b * sk, v.shape[1], d)
        out = torch.empty(b, sq, h, d, dtype=q.dtype, device=dev).transpose(1, 2)
        o3, q_step, k_step = out.transpose(1, 2).view(b * sq, h, d), sq, sk
    q_start, q_len, k_start, k_len = _seq_index(b, q_step, sq, k_step, sk, dev)
    bias = None
    if attention_mask is not None:
        lens = _prefix_lengths(attention_mask, b, sk, dev)
        if lens is not None:
            k_len = lens
        else:
            bias = _additive_mask(attention_mask, b, h, sq, sk, q.dtype)
    ops.prefill(q3, k3, v3, q_start, q_len, k_start, k_len, sq, causal, out=o3, mask=bias)
    return out


class CausalSelfAttentionBase(nn.Module):
    """Marker base, as src/nano_inference/layers/attention.py:53-75."""


class PagedCausalSelfAttention(CausalSelfAttentionBase):
    """Paged GQA self-attention whose attention core runs on the gfx950 kernels.

    Constructor and parameter names follow src/nano_inference/layers/attention.py:
    81-140 (q_proj, k_proj, v_proj, o_proj, q_norm, k_norm, rotary), so the
    reference's model code and state dicts use it unchanged.
    """

    def __init__(
        self,
        hidden_size: int,
        num_heads: int,
        num_kv_heads: Optional[int] = None,
        head_dim: Optional[int] = None,
        use_qk_norm: bool = False,
        qkv_bias: bool = False,
        out_bias: bool = False,
        rope_base: float = 10000.0,
    ):
        super().__init__()
        if head_dim is None and hidden_size % num_heads != 0:
            raise ValueError(
                f"hidden_size must be divisible by num_heads, got {hidden_size=} and {num_heads=}"
            )
        if num_kv_heads is None:
            num_kv_heads = num_heads
        if num_heads % num_kv_heads != 0:
            raise ValueError(
                f"num_heads must be divisible by num_kv_heads, got {num_heads=} and {num_kv_heads=}"
            )
        self.hidden_size = hidden_size
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim if head_dim is not None else hidden_size // num_heads
        self.use_qk_norm = use_qk_norm
        hd = self.head_dim
        self.q_proj = nn.Linear(hidden_size, num_heads * hd, bias=qkv_bias)
        self.k_proj = nn.Linear(hidden_size, num_kv_heads * hd, bias=qkv_bias)
        self.v_proj = nn.Linear(hidden_size, num_kv_heads * hd, bias=qkv_bias)
        self.o_proj = nn.Linear(num_heads * hd, hidden_size, bias=out_bias)
        self.q_norm = RMSNorm(hd) if use_qk_norm else None
        self.k_norm = RMSNorm(hd) if use_qk_norm else None
        self.rotary = RotaryEmbedding(head_dim=hd, base=rope_base)
        self.layer_idx: Optional[int] = None
        # QK-norm, RoPE and the cache write in one fused kernel (head_dim 128 on the
        # GPU); False keeps the PyTorch ops.
        self.fused_qk = True

    def _apply_rotary(self, q, k, position_ids, metadata=None) -> Tuple[torch.Tensor, torch.Tensor]:
        return self.rotary(q, k, position_ids)

    def _rope_positions(self, position_ids, metadata):
        """(positions, mrope_section) for the fused kernel: 1-D RoPE here."""
        return position_ids, None

    def _scales(self, metadata):
        """This layer's fp8 row scales (None for caches in the model dtype)."""
        if metadata is None or metadata.k_scale is None or metadata.v_scale is None:
            return None, None
        return metadata.k_scale[self.layer_idx], metadata.v_scale[self.layer_idx]

    def _qkv(self, x, position_ids, metadata, k_cache=None, v_cache=None):
        """Projected, normalised and rotated q, k and v; the last item tells whether
        k/v were also written to (k_cache, v_cache) through the metadata's slots."""
        b, s, _ = x.shape
        q = self.q_proj(x).view(b, s, self.num_heads, self.head_dim)
        k = self.k_proj(x).view(b, s, self.num_kv_heads, self.head_dim)
        v = self.v_proj(x).view(b, s, self.num_kv_heads, self.head_dim)
        if self.fused_qk and x.is_cuda and self.head_dim == 128 and \
                x.dtype in (torch.bfloat16, torch.float32):
            pos, section = self._rope_positions(position_ids, metadata)
            write = k_cache is not None and metadata is not None and \
                metadata.slot_mapping is not None
            norm = self.q_norm is not None
            ks, vs = self._scales(metadata) if write else (None, None)
            ops.qk_norm_rope_kv_write(
                q, k, v, self.q_norm.weight if norm else None,
                self.k_norm.weight if norm else None, self.q_norm.eps if norm else 0.0,
                pos, self.rotary.inv_freq, section,
                k_cache if write else None, v_cache if write else None,
                metadata.slot_mapping if write else None, ks, vs)
            return q, k, v, write
        if self.q_norm is not None:
            q = self.q_norm(q)
        if self.k_norm is not None:
            k = self.k_norm(k)
        q, k = self._apply_rotary(q, k, position_ids, metadata)
        return q, k, v, False

    def _dense_causal(self, q, k, v, attention_mask):
        """No-cache path (metadata None): causal attention over the step's K/V."""
        b, s = q.shape[:2]
        dev = q.device
        ar, lens, _, k_len = _seq_index(b, s, s, s, s, dev)
        bias = None
        if attention_mask is not None:
            plen = _prefix_lengths(attention_mask, b, s, dev)
            if plen is not None:
                k_len = plen
            else:
                bias = _additive_mask(attention_mask, b, self.num_heads, s, s, q.dtype)
        return ops.prefill(
            q.reshape(b * s, self.num_heads, self.head_dim),
            k.reshape(b * s, self.num_kv_heads, self.head_dim),
            v.reshape(b * s, self.num_kv_heads, self.head_dim),
            ar, lens, ar, k_len, s, ops.CAUSAL_TOP_LEFT, mask=bias,
        )

    def forward(
        self,
        x: torch.Tensor,
        position_ids: torch.Tensor,
        attention_mask: Optional[torch.Tensor] = None,
        metadata: Optional[AttentionMetadata] = None,
    ) -> torch.Tensor:
        b, s, _ = x.shape
        if metadata is None:
            q, k, v, _ = self._qkv(x, position_ids, None)
            attn = self._dense_causal(q, k, v, attention_mask)
            return self.o_proj(attn.view(b, s, self.num_heads * self.head_dim))
        assert self.layer_idx is not None, "layer_idx must be set for PagedCausalSelfAttention"

        k_cache = v_cache = None
        if metadata.k_cache is not None and metadata.v_cache is not None:
            k_cache = metadata.k_cache[self.layer_idx]
            v_cache = metadata.v_cache[self.layer_idx]
        q, k, v, written = self._qkv(x, position_ids, metadata, k_cache, v_cache)

        # 1. KV write (src/nano_inference/layers/attention.py:267-278), unless the
        # fused QK kernel already wrote the step's rows.
        ks, vs = self._scales(metadata)
        if not written and k_cache is not None and metadata.slot_mapping is not None:
            ops.kv_write(k, v, k_cache, v_cache, metadata.slot_mapping, ks, vs)

        if isinstance(metadata, PackedAttentionMetadata):
            attn = self._packed_attention(q, k_cache, v_cache, metadata, ks, vs)
        elif metadata.is_prefill:
            # 2a. Prefill attends over the step's fresh K/V (:281-284).  Padded
            # rows past a sequence's length see all its keys, as in the reference.
            attn = self._dense_causal(q, k, v, attention_mask)
        elif k_cache is not None and metadata.kv_block_tables is not None \
                and metadata.context_lens is not None:
            bt = metadata.kv_block_tables
            ctx = metadata.context_lens
            if s == 1:
                # 2b. Decode: gather + GQA + mask + softmax in one kernel (:285-332).
                attn = ops.paged_decode(q[:, 0], k_cache, v_cache, bt, ctx, k_scale=ks,
                                        v_scale=vs, workspace=metadata.decode_workspace)
            else:
                # 2c. Several new tokens on top of cached context: chunked prefill.
                dev = x.device
                q_len = (metadata.slot_mapping >= 0).sum(dim=1).to(torch.int32)
                q_start = torch.arange(b, device=dev, dtype=torch.int32) * s
                attn = torch.zeros(b * s, self.num_heads, self.head_dim, dtype=q.dtype,
                                   device=dev)
                ops.prefill_paged(q.reshape(b * s, self.num_heads, self.head_dim), k_cache,
                                  v_cache, bt, q_start, q_len, ctx, s,
                                  ops.CAUSAL_BOTTOM_RIGHT, out=attn, k_scale=ks, v_scale=vs)
        else:
            attn = self._dense_causal(q, k, v, attention_mask)
        return self.o_proj(attn.reshape(b, s, self.num_heads * self.head_dim))


    def _packed_attention(self, q, k_cache, v_cache, md: PackedAttentionMetadata, ks=None,
                          vs=None):
        """Decode rows through the decode kernel, chunk rows through the chunked
        prefill kernel, both reading the paged cache the step has just written."""
        if k_cache is None:
            raise ValueError("a packed step needs the KV cache")
        t = q.shape[0] * q.shape[1]
        q2 = q.reshape(t, self.num_heads, self.head_dim)
        out = torch.empty_like(q2)
        nd = md.num_decode
        n = md.q_start.shape[0]
        if nd > 0:
            ops.paged_decode(q2[:nd], k_cache, v_cache, md.kv_block_tables[:nd],
                             md.context_lens[:nd], out=out[:nd], k_scale=ks, v_scale=vs,
                             workspace=md.decode_workspace)
        if nd < n:
            ops.prefill_paged(q2, k_cache, v_cache, md.kv_block_tables[nd:], md.q_start[nd:],
                              md.q_len[nd:], md.context_lens[nd:], md.max_q_len,
                              ops.CAUSAL_BOTTOM_RIGHT, out=out, k_scale=ks, v_scale=vs)
        return out


class Qwen25VLDecoderAttention(PagedCausalSelfAttention):
    """PagedCausalSelfAttention with 3-axis mRoPE (src/nano_inference/layers/attention.py:343-371)."""

    def __init__(self, *args, mrope_section=(16, 24, 24), **kwargs):
        super().__init__(*args, **kwargs)
        self.rotary = MRotaryEmbedding(head_dim=self.head_dim, base=self.rotary.base,
                                       mrope_section=mrope_section)

    def _mrope_ids(self, position_ids, metadata):
        if metadata is not None and metadata.mrope_position_ids is not None:
            return metadata.mrope_position_ids
        return position_ids.unsqueeze(0).expand(3, -1, -1)

    def _apply_rotary(self, q, k, position_ids, metadata=None):
        return self.rotary(q, k, self._mrope_ids(position_ids, metadata))

    def _rope_positions(self, position_ids, metadata):
        return self._mrope_ids(position_ids, metadata), self.rotary._section_freqs
