"""Tensor-level wrappers of the gfx950 attention kernels.

Each function validates shapes, dtypes and devices on the host (raising
ValueError, as the reference layers do for bad configurations,
src/nano_inference/layers/attention.py:105-116), then calls one C-ABI entry
point of libnia_attn.so on the current HIP stream.  A nonzero status raises
``NiaError`` (a RuntimeError).  Nothing here computes attention itself.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from . import _lib
from ._lib import CAUSAL_BOTTOM_RIGHT, CAUSAL_NONE, CAUSAL_TOP_LEFT  # noqa: F401

_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32}


def _dtype_code(t: torch.Tensor, allowed=(torch.bfloat16, torch.float32)) -> int:
    if t.dtype not in allowed:
        raise ValueError(f"unsupported dtype {t.dtype}; expected one of {allowed}")
    return _DTYPES[t.dtype]


def _require_gpu(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    for t in tensors:
        if t.device.type != "cuda":
            raise ValueError(
                f"attention kernels run on the GPU only; got a tensor on {t.device}"
            )
        if t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _last_contig(name: str, t: torch.Tensor) -> None:
    if t.stride(-1) != 1:
        raise ValueError(f"{name} must have a contiguous last dimension")


def _default_scale(head_dim: int, scale: Optional[float]) -> float:
    # The reference divides the scores by sqrt(head_dim) (attention.py:27).
    return 1.0 / math.sqrt(head_dim) if scale is None else float(scale)


# ---------------------------------------------------------------------------------
# KV-cache write
# ---------------------------------------------------------------------------------


FP8_CACHE_DTYPES = (torch.uint8, torch.float8_e4m3fn)


def is_fp8_cache(cache: torch.Tensor) -> bool:
    """True for a cache in the fp8 format (e4m3 codes, one fp32 scale per row)."""
    return cache.dtype in FP8_CACHE_DTYPES


def _fp8_scales(k_cache, k_scale, v_scale) -> Tuple[torch.Tensor, torch.Tensor]:
    if k_scale is None or v_scale is None:
        raise ValueError("an fp8 cache needs k_scale and v_scale")
    shape = tuple(k_cache.shape[:3])
    for name, t in (("k_scale", k_scale), ("v_scale", v_scale)):
        if t.dtype != torch.float32 or tuple(t.shape) != shape or not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous float32 {shape}")
        if t.device != k_cache.device:
            raise ValueError(f"{name} must be on the cache's device")
    return k_scale, v_scale


def kv_write(
    k: torch.Tensor,
    v: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_scale: Optional[torch.Tensor] = None,
    v_scale: Optional[torch.Tensor] = None,
) -> None:
    """Scatter new K/V rows into one layer's paged cache, in place.

    Same effect as the loop at src/nano_inference/layers/attention.py:267-278:
    for every token t with ``slot = slot_mapping[t] >= 0``,
    ``k_cache[slot // BS, :, slot % BS, :] = k[t]`` (and likewise for v), bit-exact.
    With fp8 caches (uint8 or float8_e4m3fn) each row is stored as e4m3 codes with
    one fp32 scale in ``k_scale`` / ``v_scale`` [num_blocks, H_kv, BS] (scale =
    max |x| / 448, code = e4m3(x / scale)).

    k, v: (..., H_kv, D) - leading dims are flattened to tokens in the order of
    ``slot_mapping.reshape(-1)``; k_cache, v_cache: [num_blocks, H_kv, BS, D].
    """
    dev = _require_gpu(k, v, k_cache, v_cache, slot_mapping)
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("k_cache/v_cache must be [num_blocks, H_kv, block_size, head_dim]")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("k_cache/v_cache layer slices must be contiguous")
    nb, hkv, bs, d = k_cache.shape
    if k.shape[-2:] != (hkv, d) or v.shape[-2:] != (hkv, d):
        raise ValueError(f"k/v trailing shape must be ({hkv}, {d}), got {tuple(k.shape)}")
    fp8 = is_fp8_cache(k_cache)
    if fp8:
        if v_cache.dtype != k_cache.dtype or k.dtype != v.dtype:
            raise ValueError("k and v (and the two caches) must share one dtype")
        k_scale, v_scale = _fp8_scales(k_cache, k_scale, v_scale)
    elif not (k.dtype == v.dtype == k_cache.dtype == v_cache.dtype):
        raise ValueError("k, v and the caches must share one dtype")
    if slot_mapping.dtype != torch.int64:
        raise ValueError("slot_mapping must be int64 (the context builder's dtype)")
    dt = _dtype_code(k)
    k2 = k.reshape(-1, hkv, d)
    v2 = v.reshape(-1, hkv, d)
    _last_contig("k", k2)
    _last_contig("v", v2)
    slots = slot_mapping.reshape(-1).contiguous()
    if slots.numel() != k2.shape[0]:
        raise ValueError(f"{slots.numel()} slots for {k2.shape[0]} tokens")
    lib = _lib.load()
    if fp8:
        st = lib.nia_kv_write_fp8(
            k2.data_ptr(), k2.stride(0), k2.stride(1),
            v2.data_ptr(), v2.stride(0), v2.stride(1),
            k_cache.data_ptr(), v_cache.data_ptr(), k_scale.data_ptr(), v_scale.data_ptr(),
            slots.data_ptr(), k2.shape[0], hkv, d, bs, nb, dt, _stream(dev),
        )
        _lib.check("nia_kv_write_fp8", st)
        return
    st = lib.nia_kv_write(
        k2.data_ptr(), k2.stride(0), k2.stride(1),
        v2.data_ptr(), v2.stride(0), v2.stride(1),
        k_cache.data_ptr(), v_cache.data_ptr(), slots.data_ptr(),
        k2.shape[0], hkv, d, bs, nb, dt, _stream(dev),
    )
    _lib.check("nia_kv_write", st)


# ---------------------------------------------------------------------------------
# Paged decode
# ---------------------------------------------------------------------------------


def decode_workspace_bytes(batch: int, num_heads: int, num_kv_heads: int, max_blocks: int,
                           block_size: int, head_dim: int, dtype=torch.bfloat16) -> int:
    """Bytes of decode workspace a call with these sizes needs (``dtype``: the query
    dtype; fp8 caches take bf16 queries)."""
    return int(
        _lib.load().nia_paged_decode_workspace_size(batch, num_heads, num_kv_heads, max_blocks,
                                                    block_size, head_dim,
                                                    _dtype_code_of(dtype)))


def _dtype_code_of(dtype) -> int:
    if dtype not in _DTYPES:
        raise ValueError(f"unsupported dtype {dtype}")
    return _DTYPES[dtype]


def check_decode_shape(head_dim: int, block_size: int, num_heads: int, num_kv_heads: int,
                       dtype=torch.bfloat16, fp8_cache: bool = False) -> None:
    """Raise ValueError unless paged decode supports this layout (the limits of
    include/nia_attn.h): bf16 - block size a power of two >= 4, head_dim 64 / 80 / 96 /
    128, at most 16 query heads per KV head; fp8 caches - head_dim 128, block size a
    power of two >= 16; fp32 - head_dim 64 / 80 / 96 / 128, any block size and group.
    A KV pool can be checked when it is built, before any step runs."""
    if num_kv_heads <= 0 or num_heads % num_kv_heads != 0:
        raise ValueError(f"num_heads must be divisible by num_kv_heads, got {num_heads=} and "
                         f"{num_kv_heads=}")
    if head_dim not in (64, 80, 96, 128):
        raise ValueError(f"paged decode supports head_dim 64, 80, 96 or 128, not {head_dim}")
    if block_size <= 0:
        raise ValueError(f"block_size must be positive, got {block_size}")
    if dtype == torch.float32 and not fp8_cache:
        return
    pow2 = block_size & (block_size - 1) == 0
    if fp8_cache:
        if head_dim != 128 or not pow2 or block_size < 16:
            raise ValueError("fp8 KV caches need head_dim 128 and a power-of-two block size "
                             f">= 16 (got head_dim {head_dim}, block_size {block_size})")
    elif not pow2 or block_size < 4:
        raise ValueError("bf16 paged decode needs a power-of-two block size >= 4, "
                         f"got {block_size}")
    if num_heads // num_kv_heads > 16:
        raise ValueError("bf16 paged decode takes at most 16 query heads per KV head, got "
                         f"{num_heads // num_kv_heads}")


# One workspace per (device, stream): calls on one stream run one after another and may
# share it; calls on other streams get their own.  A workspace that is outgrown is kept
# (in _RETIRED) rather than freed, since a captured HIP graph may still hold its address.
_DECODE_WS: dict = {}
_RETIRED: list = []


def decode_workspace(device: torch.device, nbytes: int, stream=None) -> torch.Tensor:
    """A decode workspace of at least ``nbytes`` for (``device``, ``stream``) (default: the
    device's current stream), cached and reused by later calls on that stream."""
    dev = torch.device(device)
    st = torch.cuda.current_stream(dev) if stream is None else stream
    key = (dev, st.cuda_stream)
    ws = _DECODE_WS.get(key)
    if ws is None or ws.numel() < nbytes:
        if ws is not None:
            _RETIRED.append(ws)
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
        _DECODE_WS[key] = ws
    return ws


def paged_decode(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    scale: Optional[float] = None,
    out: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
    k_scale: Optional[torch.Tensor] = None,
    v_scale: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """One query token per sequence against its paged keys.

    Same result as the decode branch of src/nano_inference/layers/attention.py:285-332
    for S_step = 1.  q: (B, H, D) or (B, 1, H, D); k_cache/v_cache: one layer,
    [num_blocks, H_kv, BS, D]; block_tables: (B, max_blocks) int32;
    context_lens: (B,) int64.  Returns (B, H, D) (or q's 4-D shape).
    ``workspace`` (optional, uint8, at least ``decode_workspace_bytes(...)``); by
    default the cached one of the current stream (``decode_workspace``) is used.
    fp8 caches (uint8 / float8_e4m3fn codes) take their per-row ``k_scale`` /
    ``v_scale`` [num_blocks, H_kv, BS] float32 and bf16 queries.
    """
    dev = _require_gpu(q, k_cache, v_cache, block_tables, context_lens)
    squeeze = q.dim() == 4
    if squeeze:
        if q.shape[1] != 1:
            raise ValueError("paged_decode takes one query token per sequence")
        q3 = q[:, 0]
    elif q.dim() == 3:
        q3 = q
    else:
        raise ValueError(f"q must be (B, H, D) or (B, 1, H, D), got {tuple(q.shape)}")
    b, h, d = q3.shape
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("k_cache/v_cache must be [num_blocks, H_kv, block_size, head_dim]")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("k_cache/v_cache layer slices must be contiguous")
    nb, hkv, bs, dc = k_cache.shape
    if dc != d:
        raise ValueError(f"head_dim mismatch: q {d}, cache {dc}")
    if h % hkv != 0:
        raise ValueError(f"num_heads must be divisible by num_kv_heads, got {h=} and {hkv=}")
    fp8 = is_fp8_cache(k_cache)
    if fp8:
        if v_cache.dtype != k_cache.dtype or q3.dtype != torch.bfloat16:
            raise ValueError("fp8 caches take bf16 queries (and share one dtype)")
        k_scale, v_scale = _fp8_scales(k_cache, k_scale, v_scale)
    elif not (q3.dtype == k_cache.dtype == v_cache.dtype):
        raise ValueError("q and the caches must share one dtype")
    if block_tables.dtype != torch.int32 or block_tables.dim() != 2 or block_tables.shape[0] != b:
        raise ValueError("block_tables must be (B, max_blocks) int32")
    if context_lens.dtype != torch.int64 or context_lens.shape != (b,):
        raise ValueError("context_lens must be (B,) int64")
    if block_tables.stride(1) != 1:
        block_tables = block_tables.contiguous()
    context_lens = context_lens.contiguous()
    dt = _dtype_code(q3)
    _last_contig("q", q3)
    if out is None:
        out3 = torch.empty((b, h, d), dtype=q3.dtype, device=dev)
    else:
        out3 = out[:, 0] if out.dim() == 4 else out
        if out3.shape != (b, h, d) or out3.dtype != q3.dtype:
            raise ValueError("out must match q's shape and dtype")
        _last_contig("out", out3)
    max_blocks = block_tables.shape[1]
    check_decode_shape(d, bs, h, hkv, q3.dtype, fp8)
    need = decode_workspace_bytes(b, h, hkv, max_blocks, bs, d, q3.dtype)
    if workspace is None:
        workspace = decode_workspace(dev, need)
    ws_bytes = workspace.numel() * workspace.element_size()
    if ws_bytes < need:
        raise ValueError(f"decode workspace of {ws_bytes} bytes, {need} needed")
    ws_ptr = workspace.data_ptr()
    lib = _lib.load()
    if fp8:
        st = lib.nia_paged_decode_fp8(
            out3.data_ptr(), out3.stride(0), out3.stride(1),
            q3.data_ptr(), q3.stride(0), q3.stride(1),
            k_cache.data_ptr(), v_cache.data_ptr(), k_scale.data_ptr(), v_scale.data_ptr(),
            block_tables.data_ptr(), block_tables.stride(0), max_blocks, context_lens.data_ptr(),
            b, h, hkv, d, bs, nb, _default_scale(d, scale), ws_ptr, ws_bytes, _stream(dev),
        )
        _lib.check("nia_paged_decode_fp8", st)
    else:
        st = lib.nia_paged_decode(
            out3.data_ptr(), out3.stride(0), out3.stride(1),
            q3.data_ptr(), q3.stride(0), q3.stride(1),
            k_cache.data_ptr(), v_cache.data_ptr(),
            block_tables.data_ptr(), block_tables.stride(0), max_blocks,
            context_lens.data_ptr(), b, h, hkv, d, bs, nb, _default_scale(d, scale), ws_ptr,
            ws_bytes, dt, _stream(dev),
        )
        _lib.check("nia_paged_decode", st)
    if out is not None:
        return out
    return out3.unsqueeze(1) if squeeze else out3


# ---------------------------------------------------------------------------------
# Prefill (contiguous K/V) and varlen
# ---------------------------------------------------------------------------------


def _i32(name: str, t: torch.Tensor, n: int) -> torch.Tensor:
    if t.dim() != 1 or t.shape[0] != n:
        raise ValueError(f"{name} must be ({n},)")
    return t.to(torch.int32).contiguous()


def prefill(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    q_start: torch.Tensor,
    q_len: torch.Tensor,
    k_start: torch.Tensor,
    k_len: torch.Tensor,
    max_q_len: int,
    causal: int = CAUSAL_TOP_LEFT,
    scale: Optional[float] = None,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Varlen attention over contiguous K/V rows (nia_prefill), bf16 or fp32.

    q/out: (Tq, H, D); k/v: (Tk, H_kv, D), each with a contiguous last dim.
    Sequence s owns query rows q_start[s] .. + q_len[s] and key rows
    k_start[s] .. + k_len[s].  ``causal`` is CAUSAL_NONE / CAUSAL_TOP_LEFT /
    CAUSAL_BOTTOM_RIGHT (see include/nia_attn.h).
    """
    dev = _require_gpu(q, k, v, q_start, q_len, k_start, k_len)
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3 or k.shape != v.shape:
        raise ValueError("q must be (Tq, H, D) and k, v (Tk, H_kv, D)")
    _, h, d = q.shape
    hkv = k.shape[1]
    if k.shape[2] != d:
        raise ValueError("head_dim mismatch between q and k/v")
    if h % hkv != 0:
        raise ValueError(f"num_heads must be divisible by num_kv_heads, got {h=} and {hkv=}")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("q, k and v must share one dtype")
    dt = _dtype_code(q)
    for name, t in (("q", q), ("k", k), ("v", v)):
        _last_contig(name, t)
    n = q_start.shape[0]
    qs, ql, ks, kl = (_i32(nm, t, n) for nm, t in
                      (("q_start", q_start), ("q_len", q_len), ("k_start", k_start),
                       ("k_len", k_len)))
    if out is None:
        out = torch.empty_like(q, memory_format=torch.contiguous_format)
    elif out.shape != q.shape or out.dtype != q.dtype:
        raise ValueError("out must match q's shape and dtype")
    _last_contig("out", out)
    lib = _lib.load()
    st = lib.nia_prefill(
        out.data_ptr(), out.stride(0), out.stride(1),
        q.data_ptr(), q.stride(0), q.stride(1),
        k.data_ptr(), k.stride(0), k.stride(1),
        v.data_ptr(), v.stride(0), v.stride(1),
        qs.data_ptr(), ql.data_ptr(), ks.data_ptr(), kl.data_ptr(),
        n, int(max_q_len), h, hkv, d, _default_scale(d, scale), int(causal), dt, _stream(dev),
    )
    _lib.check("nia_prefill", st)
    return out


def varlen_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: Optional[torch.Tensor] = None,
    max_seqlen_q: Optional[int] = None,
    causal: bool = False,
    scale: Optional[float] = None,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Packed varlen attention with cu_seqlens (vision tower: causal=False).

    Chunk i owns rows cu_seqlens[i] .. cu_seqlens[i+1]; causal=True aligns the
    mask top-left (equal q/k lengths in the prefill case).  ``max_seqlen_q``
    sizes the launch grid; when omitted it is read back from the device.
    """
    if cu_seqlens_k is None:
        cu_seqlens_k = cu_seqlens_q
    cq = cu_seqlens_q.to(torch.int32)
    ck = cu_seqlens_k.to(torch.int32)
    lq = cq[1:] - cq[:-1]
    lk = ck[1:] - ck[:-1]
    if max_seqlen_q is None:
        max_seqlen_q = int(lq.max().item()) if lq.numel() else 0
    return prefill(q, k, v, cq[:-1], lq, ck[:-1], lk, max_seqlen_q,
                   CAUSAL_TOP_LEFT if causal else CAUSAL_NONE, scale, out)


# ---------------------------------------------------------------------------------
# Chunked prefill over the paged cache
# ---------------------------------------------------------------------------------


def prefill_paged(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    q_start: torch.Tensor,
    q_len: torch.Tensor,
    context_lens: torch.Tensor,
    max_q_len: int,
    causal: int = CAUSAL_BOTTOM_RIGHT,
    scale: Optional[float] = None,
    out: Optional[torch.Tensor] = None,
    k_scale: Optional[torch.Tensor] = None,
    v_scale: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Query chunks against their paged keys (nia_prefill_paged), bf16 or fp32.

    q/out: (Tq, H, D).  Sequence s has q_len[s] query rows starting at token
    q_start[s], sitting at absolute positions context_lens[s] - q_len[s] + j,
    and reads keys [0, context_lens[s]) through block_tables (B, max_blocks) int32.
    fp8 caches (with ``k_scale`` / ``v_scale``): the keys are first dequantised into
    contiguous bf16 rows (nia_dequant_gather_fp8), then attended by nia_prefill.
    """
    if is_fp8_cache(k_cache):
        return _prefill_paged_fp8(q, k_cache, v_cache, block_tables, q_start, q_len,
                                   context_lens, max_q_len, causal, scale, out, k_scale, v_scale)
    dev = _require_gpu(q, k_cache, v_cache, block_tables, q_start, q_len, context_lens)
    if q.dim() != 3:
        raise ValueError("q must be (Tq, H, D)")
    _, h, d = q.shape
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("k_cache/v_cache must be [num_blocks, H_kv, block_size, head_dim]")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("k_cache/v_cache layer slices must be contiguous")
    nb, hkv, bs, dc = k_cache.shape
    if dc != d:
        raise ValueError("head_dim mismatch between q and the cache")
    if h % hkv != 0:
        raise ValueError(f"num_heads must be divisible by num_kv_heads, got {h=} and {hkv=}")
    if not (q.dtype == k_cache.dtype == v_cache.dtype):
        raise ValueError("q and the caches must share one dtype")
    dt = _dtype_code(q)
    _last_contig("q", q)
    n = q_start.shape[0]
    if block_tables.dtype != torch.int32 or block_tables.dim() != 2 or block_tables.shape[0] != n:
        raise ValueError("block_tables must be (B, max_blocks) int32")
    if block_tables.stride(1) != 1:
        block_tables = block_tables.contiguous()
    if context_lens.dtype != torch.int64 or context_lens.shape != (n,):
        raise ValueError("context_lens must be (B,) int64")
    qs, ql = _i32("q_start", q_start, n), _i32("q_len", q_len, n)
    context_lens = context_lens.contiguous()
    if out is None:
        out = torch.empty_like(q, memory_format=torch.contiguous_format)
    elif out.shape != q.shape or out.dtype != q.dtype:
        raise ValueError("out must match q's shape and dtype")
    _last_contig("out", out)
    lib = _lib.load()
    st = lib.nia_prefill_paged(
        out.data_ptr(), out.stride(0), out.stride(1),
        q.data_ptr(), q.stride(0), q.stride(1),
        k_cache.data_ptr(), v_cache.data_ptr(),
        block_tables.data_ptr(), block_tables.stride(0), block_tables.shape[1],
        qs.data_ptr(), ql.data_ptr(), context_lens.data_ptr(),
        n, int(max_q_len), h, hkv, d, bs, nb, _default_scale(d, scale), int(causal), dt,
        _stream(dev),
    )
    _lib.check("nia_prefill_paged", st)
    return out


def _prefill_paged_fp8(q, k_cache, v_cache, block_tables, q_start, q_len, context_lens,
                       max_q_len, causal, scale, out, k_scale, v_scale):
    dev = _require_gpu(q, k_cache, v_cache, block_tables, q_start, q_len, context_lens)
    if q.dim() != 3 or k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("q must be (Tq, H, D), caches [num_blocks, H_kv, block_size, D]")
    if v_cache.dtype != k_cache.dtype or q.dtype != torch.bfloat16:
        raise ValueError("fp8 caches take bf16 queries (and share one dtype)")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("k_cache/v_cache layer slices must be contiguous")
    k_scale, v_scale = _fp8_scales(k_cache, k_scale, v_scale)
    nb, hkv, bs, d = k_cache.shape
    n = q_start.shape[0]
    if block_tables.dtype != torch.int32 or block_tables.dim() != 2 or block_tables.shape[0] != n:
        raise ValueError("block_tables must be (B, max_blocks) int32")
    if block_tables.stride(1) != 1:
        block_tables = block_tables.contiguous()
    if context_lens.dtype != torch.int64 or context_lens.shape != (n,):
        raise ValueError("context_lens must be (B,) int64")
    context_lens = context_lens.contiguous()
    mb = block_tables.shape[1]
    stride = mb * bs
    keys = torch.empty((n * stride, hkv, d), dtype=torch.bfloat16, device=dev)
    vals = torch.empty_like(keys)
    lib = _lib.load()
    st = lib.nia_dequant_gather_fp8(
        k_cache.data_ptr(), v_cache.data_ptr(), k_scale.data_ptr(), v_scale.data_ptr(),
        block_tables.data_ptr(), block_tables.stride(0), mb, context_lens.data_ptr(), n, hkv, d,
        bs, nb, keys.data_ptr(), vals.data_ptr(), stride, _stream(dev))
    _lib.check("nia_dequant_gather_fp8", st)
    k_start = torch.arange(n, device=dev, dtype=torch.int32) * stride
    k_len = context_lens.clamp(0, stride).to(torch.int32)
    return prefill(q, keys, vals, q_start, q_len, k_start, k_len, max_q_len, causal, scale, out)


# ---------------------------------------------------------------------------------
# Fused QK-RMSNorm + RoPE / mRoPE + KV write
# ---------------------------------------------------------------------------------


def qk_norm_rope_kv_write(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    q_norm_weight: Optional[torch.Tensor],
    k_norm_weight: Optional[torch.Tensor],
    eps: float,
    positions: torch.Tensor,
    inv_freq: torch.Tensor,
    mrope_section: Optional[Tuple[int, int, int]] = None,
    k_cache: Optional[torch.Tensor] = None,
    v_cache: Optional[torch.Tensor] = None,
    slot_mapping: Optional[torch.Tensor] = None,
    k_scale: Optional[torch.Tensor] = None,
    v_scale: Optional[torch.Tensor] = None,
) -> None:
    """QK-RMSNorm, RoPE (or mRoPE) in place on q and k, then the KV-cache write
    (fp8 caches: e4m3 codes plus the per-row ``k_scale`` / ``v_scale``, as kv_write).

    Same values as ``q_norm(q)``, ``k_norm(k)``, the rotary module and the write loop
    of src/nano_inference/layers/attention.py:254-278 (every intermediate rounded to
    the model dtype as the PyTorch ops round it).
    q: (..., H, 128); k, v: (..., H_kv, 128) with the same leading dims (tokens);
    positions: the leading dims' position ids, or (3, *leading) for mRoPE with
    ``mrope_section``; inv_freq: (64,) (any float dtype); norm weights (128,) or None (no QK
    norm; both or neither); caches one layer [num_blocks, H_kv, BS, 128] or None.
    """
    dev = _require_gpu(q, k, v, positions, inv_freq)
    d = q.shape[-1]
    if k.shape[-1] != d or v.shape != k.shape or q.shape[:-2] != k.shape[:-2]:
        raise ValueError("q (..., H, D), k and v (..., H_kv, D) with the same leading dims")
    if (q_norm_weight is None) != (k_norm_weight is None):
        raise ValueError("q and k norm weights must both be given or both be None")
    dt = _dtype_code(q)
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("q, k and v must share one dtype")
    lead = q.shape[:-2]
    n = math.prod(lead)
    try:  # q and k are updated in place, so they must be viewable as (tokens, heads, D)
        q2 = q.view(n, q.shape[-2], d)
        k2 = k.view(n, k.shape[-2], d)
    except RuntimeError as e:
        raise ValueError(f"q and k must be viewable as (tokens, heads, D): {e}") from None
    v2 = v.reshape(n, v.shape[-2], d)
    for name, t in (("q", q2), ("k", k2), ("v", v2)):
        _last_contig(name, t)
    if mrope_section is None:
        if positions.shape != lead:
            raise ValueError(f"positions must have shape {tuple(lead)}")
        num_axes, sec0, sec1 = 1, 0, 0
    else:
        if positions.shape != (3, *lead):
            raise ValueError(f"mRoPE positions must have shape (3, {tuple(lead)})")
        num_axes, sec0, sec1 = 3, int(mrope_section[0]), int(mrope_section[1])
    pos = positions.reshape(num_axes, n).to(torch.int64).contiguous()
    if not inv_freq.is_floating_point() or inv_freq.numel() != d // 2:
        raise ValueError(f"inv_freq must be a ({d // 2},) floating-point table")
    # A module cast to the model dtype holds a rounded table; the products
    # position * inv_freq are still formed in fp32 from those rounded values.
    inv = inv_freq.to(torch.float32).contiguous()
    qw = kw = None
    if q_norm_weight is not None:
        if q_norm_weight.shape != (d,) or k_norm_weight.shape != (d,) or \
                q_norm_weight.dtype != q.dtype or k_norm_weight.dtype != q.dtype:
            raise ValueError(f"norm weights must be ({d},) in the model dtype")
        qw, kw = q_norm_weight.contiguous(), k_norm_weight.contiguous()
    kc_ptr = vc_ptr = sl_ptr = None
    bs, nb = 1, 0
    keep = []
    if k_cache is not None:
        if v_cache is None or slot_mapping is None:
            raise ValueError("a cache write needs v_cache and slot_mapping")
        if k_cache.dim() != 4 or v_cache.shape != k_cache.shape or \
                k_cache.shape[1] != k2.shape[1] or k_cache.shape[3] != d:
            raise ValueError("k_cache/v_cache must be [num_blocks, H_kv, block_size, D]")
        if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
            raise ValueError("k_cache/v_cache layer slices must be contiguous")
        fp8 = is_fp8_cache(k_cache)
        if fp8:
            if v_cache.dtype != k_cache.dtype:
                raise ValueError("k_cache and v_cache must share one dtype")
            k_scale, v_scale = _fp8_scales(k_cache, k_scale, v_scale)
        elif k_cache.dtype != q.dtype or v_cache.dtype != q.dtype:
            raise ValueError("caches must share the model dtype")
        if slot_mapping.dtype != torch.int64 or slot_mapping.numel() != n:
            raise ValueError(f"slot_mapping must be int64 with {n} entries")
        slots = slot_mapping.reshape(-1).contiguous()
        keep.append(slots)
        nb, bs = k_cache.shape[0], k_cache.shape[2]
        kc_ptr, vc_ptr, sl_ptr = k_cache.data_ptr(), v_cache.data_ptr(), slots.data_ptr()
    lib = _lib.load()
    args = (q2.data_ptr(), q2.stride(0), q2.stride(1), k2.data_ptr(), k2.stride(0), k2.stride(1),
            v2.data_ptr(), v2.stride(0), v2.stride(1),
            qw.data_ptr() if qw is not None else None, kw.data_ptr() if kw is not None else None,
            float(eps), pos.data_ptr(), pos.stride(0), num_axes, inv.data_ptr(), sec0, sec1,
            kc_ptr, vc_ptr)
    tail = (sl_ptr, n, q2.shape[1], k2.shape[1], d, bs, nb, dt, _stream(dev))
    if k_cache is not None and is_fp8_cache(k_cache):
        st = lib.nia_qk_norm_rope_kv_write_fp8(*args, k_scale.data_ptr(), v_scale.data_ptr(),
                                               *tail)
        _lib.check("nia_qk_norm_rope_kv_write_fp8", st)
        return
    st = lib.nia_qk_norm_rope_kv_write(*args, *tail)
    _lib.check("nia_qk_norm_rope_kv_write", st)
