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
    idx = tensors[0].get_device()
    for t in tensors:
        i = t.get_device()
        if i < 0:
            raise ValueError(
                f"attention kernels run on the GPU only; got a tensor on {t.device}"
            )
        if i != idx:
            raise ValueError(f"tensors on different devices: {tensors[0].device} and {t.device}")
    return tensors[0].device


def _raw_stream(index: int) -> int:
    """The current HIP stream of device ``index`` as an integer handle."""
    return torch._C._cuda_getCurrentRawStream(index)


def _stream(dev: torch.device) -> int:
    return _raw_stream(dev.index if dev.index is not None else torch.cuda.current_device())


def _last_contig(name: str, t: torch.Tensor) -> None:
    if t.stride(-1) != 1:
        raise ValueError(f"{name} must have a contiguous last dimension")


class TensorMemo:
    """Results derived from a tensor, kept while the same tensor object comes back
    unmodified (same version counter): values read back to the host, so that the layers
    of a step which share one attention mask or one cu_seqlens tensor synchronise with
    the device once instead of once per layer, and converted copies, so that a table
    every layer passes is converted once.  Holds strong references to the last ``size``
    tensors put (small ones), so that a freed tensor's memory and id cannot come back as
    a different tensor with a stale result.  Lookups are one dict probe, whatever the
    size."""

    def __init__(self, size: int = 8):
        self.size = size
        self._items: dict = {}  # (id(tensor), key) -> (tensor, version, value), oldest first

    def get(self, t: torch.Tensor, key):
        item = self._items.get((id(t), key))
        if item is not None and item[0] is t and item[1] == t._version:
            return item[2]
        return None

    def put(self, t: torch.Tensor, key, value) -> None:
        k = (id(t), key)
        self._items.pop(k, None)
        self._items[k] = (t, t._version, value)
        while len(self._items) > self.size:
            del self._items[next(iter(self._items))]


_MAX_SEQLEN = TensorMemo()
_INV_FREQ_F32 = TensorMemo(size=512)  # one table per layer (64 floats each)


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
    lib = _lib.calls()
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


def check_pool_shape(head_dim: int, block_size: int, num_heads: int, num_kv_heads: int,
                     dtype=torch.bfloat16, fp8_cache: bool = False) -> None:
    """Raise ValueError unless every kernel a paged KV pool feeds supports its layout (the
    limits of include/nia_attn.h), so that a pool can be checked when it is built, before
    any step runs:

    * bf16 and fp32 caches: head_dim 64 / 80 / 96 / 128, any block size and group;
    * fp8 caches: head_dim 128, any block size and group.

    Any positive block size is taken, as the reference's (a free integer,
    src/nano_inference/core/config.py:54; 16 is its default).  The tuned kernels find a
    key's block by a multiply-shift division: bf16 decode takes block sizes that are
    multiples of 4 (fp8: of 16), bf16 chunked prefill any size >= 2 (multiples of 4 by DMA);
    other sizes run the fp32-softmax kernel that maps every key through the table on its
    own (correct, far slower)."""
    if num_kv_heads <= 0 or num_heads <= 0 or num_heads % num_kv_heads != 0:
        raise ValueError(f"num_heads must be divisible by num_kv_heads, got {num_heads=} and "
                         f"{num_kv_heads=}")
    if head_dim not in (64, 80, 96, 128):
        raise ValueError(f"paged attention supports head_dim 64, 80, 96 or 128, not {head_dim}")
    if block_size <= 0:
        raise ValueError(f"block_size must be positive, got {block_size}")
    if fp8_cache and head_dim != 128:
        raise ValueError(f"fp8 KV caches need head_dim 128 (got head_dim {head_dim})")


def check_decode_shape(head_dim: int, block_size: int, num_heads: int, num_kv_heads: int,
                       dtype=torch.bfloat16, fp8_cache: bool = False) -> None:
    """Raise ValueError unless paged decode supports this layout: the same limits as
    ``check_pool_shape`` (decode sets the pool's tightest ones)."""
    check_pool_shape(head_dim, block_size, num_heads, num_kv_heads, dtype, fp8_cache)


# One workspace per (device, stream): calls on one stream run one after another and may
# share it; calls on other streams get their own.  A workspace that is outgrown is kept
# (in _RETIRED) rather than freed, since a captured HIP graph may still hold its address.
# Workspaces grow geometrically (at least twice the outgrown size), so the retired ones of
# a stream add up to less than its live one; release_retired_workspaces() frees them once
# the caller knows that no graph holding them will be replayed.
_DECODE_WS: dict = {}
_RETIRED: list = []
_MIN_WS_BYTES = 1 << 20


def decode_workspace(device: torch.device, nbytes: int, stream=None) -> torch.Tensor:
    """A decode workspace of at least ``nbytes`` for (``device``, ``stream``) (default: the
    device's current stream), cached and reused by later calls on that stream."""
    dev = torch.device(device)
    if stream is not None:
        handle = stream.cuda_stream
    elif dev.type == "cuda":
        handle = _raw_stream(dev.index if dev.index is not None else torch.cuda.current_device())
    else:
        handle = 0
    key = (dev.index if dev.type == "cuda" else -1, handle)
    ws = _DECODE_WS.get(key)
    if ws is None or ws.numel() < nbytes:
        size = max(nbytes, _MIN_WS_BYTES)
        if ws is not None:
            _RETIRED.append(ws)
            size = max(size, 2 * ws.numel())
        ws = torch.empty(size, dtype=torch.uint8, device=dev)
        _DECODE_WS[key] = ws
    return ws


def retired_workspace_bytes() -> int:
    """Bytes held by outgrown decode workspaces (kept for graphs that may hold them)."""
    return sum(t.numel() for t in _RETIRED)


def release_retired_workspaces() -> int:
    """Free the outgrown decode workspaces and return their total size in bytes.  Call it
    only when no captured HIP graph that ran paged_decode before the growth will be
    replayed again (for example after deleting such graphs): a replay would write to
    freed memory."""
    n = retired_workspace_bytes()
    _RETIRED.clear()
    return n


class _DecodePlan:
    """What paged_decode validated and derived for one signature of its arguments
    (shapes, strides, dtypes, devices), so that a repeated call only reads pointers."""

    __slots__ = ("squeeze", "b", "h", "d", "hkv", "bs", "nb", "max_blocks", "dt", "fp8",
                 "scale", "need", "bt_copy", "ctx_copy", "device",
                 "q_st", "out_st", "bt_st")


_DECODE_PLANS: dict = {}
_PLAN_CACHE_MAX = 256


def _decode_plan(q, k_cache, v_cache, block_tables, context_lens, scale, out, k_scale,
                 v_scale) -> _DecodePlan:
    """Full validation of a paged_decode call (raises ValueError on a bad one)."""
    _require_gpu(q, k_cache, v_cache, block_tables, context_lens)
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
        _fp8_scales(k_cache, k_scale, v_scale)
    elif not (q3.dtype == k_cache.dtype == v_cache.dtype):
        raise ValueError("q and the caches must share one dtype")
    if block_tables.dtype != torch.int32 or block_tables.dim() != 2 or block_tables.shape[0] != b:
        raise ValueError("block_tables must be (B, max_blocks) int32")
    if context_lens.dtype != torch.int64 or context_lens.shape != (b,):
        raise ValueError("context_lens must be (B,) int64")
    _last_contig("q", q3)
    if out is not None:
        out3 = out[:, 0] if out.dim() == 4 else out
        if out3.shape != (b, h, d) or out3.dtype != q3.dtype:
            raise ValueError("out must match q's shape and dtype")
        if out.get_device() != q.get_device():
            raise ValueError("out must be on q's device")
        _last_contig("out", out3)
    max_blocks = block_tables.shape[1]
    check_decode_shape(d, bs, h, hkv, q3.dtype, fp8)
    pl = _DecodePlan()
    pl.squeeze, pl.b, pl.h, pl.d, pl.hkv, pl.bs, pl.nb = squeeze, b, h, d, hkv, bs, nb
    pl.max_blocks, pl.dt, pl.fp8 = max_blocks, _dtype_code(q3), fp8
    pl.scale = _default_scale(d, scale)
    pl.need = decode_workspace_bytes(b, h, hkv, max_blocks, bs, d, q3.dtype)
    pl.bt_copy = block_tables.stride(1) != 1
    pl.ctx_copy = not context_lens.is_contiguous()
    pl.device = q.device
    # strides of the (B, H, D) views the kernel reads and writes: q[:, 0] and out[:, 0]
    # start at q's and out's first element, so a call passes their pointers directly.
    # Without `out`, a call allocates empty_like(q) (q's shape, and its layout when q is
    # dense), whose strides follow from q's: taken here from one such allocation.
    pl.q_st = q3.stride()[:2]
    if out is None:
        like = torch.empty_like(q)
        pl.out_st = (like.stride(0), like.stride(2 if squeeze else 1))
        if like.stride(-1) != 1:
            raise ValueError("q's layout gives an output without a contiguous last dimension")
    else:
        pl.out_st = out3.stride()[:2]
    pl.bt_st = max_blocks if pl.bt_copy else block_tables.stride(0)
    return pl


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

    A call is validated in full the first time its arguments' shapes, strides, dtypes
    and devices are seen; later calls with the same signature reuse that result.
    """
    dq = q.get_device()
    sig = (q.shape, q.stride(), q.dtype, dq,
           k_cache.shape, k_cache.stride(), k_cache.dtype, k_cache.get_device(),
           v_cache.shape, v_cache.stride(), v_cache.dtype, v_cache.get_device(),
           block_tables.shape, block_tables.stride(), block_tables.dtype,
           block_tables.get_device(),
           context_lens.shape, context_lens.stride(), context_lens.dtype,
           context_lens.get_device(), scale,
           None if out is None else (out.shape, out.stride(), out.dtype, out.get_device()),
           None if k_scale is None else (k_scale.shape, k_scale.stride(), k_scale.dtype,
                                         k_scale.get_device()),
           None if v_scale is None else (v_scale.shape, v_scale.stride(), v_scale.dtype,
                                         v_scale.get_device()))
    pl = _DECODE_PLANS.get(sig)
    if pl is None:
        pl = _decode_plan(q, k_cache, v_cache, block_tables, context_lens, scale, out,
                          k_scale, v_scale)
        if len(_DECODE_PLANS) >= _PLAN_CACHE_MAX:
            _DECODE_PLANS.clear()
        _DECODE_PLANS[sig] = pl
    stream = _raw_stream(dq)
    if workspace is None:
        ws = _DECODE_WS.get((dq, stream))
        if ws is None or ws.numel() < pl.need:
            ws = decode_workspace(pl.device, pl.need)
        ws_bytes = ws.numel()  # uint8
    else:
        ws = workspace
        if ws.get_device() != dq:
            raise ValueError(f"decode workspace on {ws.device}, q on {q.device}")
        ws_bytes = ws.numel() * ws.element_size()
        if ws_bytes < pl.need:
            raise ValueError(f"decode workspace of {ws_bytes} bytes, {pl.need} needed")
    if out is None:
        out3 = torch.empty_like(q)
    else:
        out3 = out
    if pl.bt_copy:
        block_tables = block_tables.contiguous()
    if pl.ctx_copy:
        context_lens = context_lens.contiguous()
    lib = _lib.calls()
    q_st, o_st = pl.q_st, pl.out_st
    if pl.fp8:
        st = lib.nia_paged_decode_fp8(
            out3.data_ptr(), o_st[0], o_st[1], q.data_ptr(), q_st[0], q_st[1],
            k_cache.data_ptr(), v_cache.data_ptr(), k_scale.data_ptr(), v_scale.data_ptr(),
            block_tables.data_ptr(), pl.bt_st, pl.max_blocks,
            context_lens.data_ptr(), pl.b, pl.h, pl.hkv, pl.d, pl.bs, pl.nb, pl.scale,
            ws.data_ptr(), ws_bytes, stream,
        )
        if st:
            _lib.check("nia_paged_decode_fp8", st)
    else:
        st = lib.nia_paged_decode(
            out3.data_ptr(), o_st[0], o_st[1], q.data_ptr(), q_st[0], q_st[1],
            k_cache.data_ptr(), v_cache.data_ptr(),
            block_tables.data_ptr(), pl.bt_st, pl.max_blocks,
            context_lens.data_ptr(), pl.b, pl.h, pl.hkv, pl.d, pl.bs, pl.nb, pl.scale,
            ws.data_ptr(), ws_bytes, pl.dt, stream,
        )
        if st:
            _lib.check("nia_paged_decode", st)
    return out3


# ---------------------------------------------------------------------------------
# Prefill (contiguous K/V) and varlen
# ---------------------------------------------------------------------------------


def _i32(name: str, t: torch.Tensor, n: int) -> torch.Tensor:
    if t.dim() != 1 or t.shape[0] != n:
        raise ValueError(f"{name} must be ({n},)")
    if t.dtype == torch.int32 and t.stride(0) == 1:
        return t
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
    mask: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Varlen attention over contiguous K/V rows (nia_prefill), bf16 or fp32.

    q/out: (Tq, H, D); k/v: (Tk, H_kv, D), each with a contiguous last dim.
    Sequence s owns query rows q_start[s] .. + q_len[s] and key rows
    k_start[s] .. + k_len[s].  ``causal`` is CAUSAL_NONE / CAUSAL_TOP_LEFT /
    CAUSAL_BOTTOM_RIGHT (see include/nia_attn.h).  ``mask`` (optional, nia_prefill_masked):
    an additive float mask indexed [sequence, head, query row, key] (size-1 dimensions
    broadcast), added to the scaled scores; -inf masks a key.
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
    if mask is not None:
        # the mask must cover every key the kernels read: one read of the key lengths (general
        # masks are rare; prefix masks take the key-length path and never come here)
        max_keys = int(kl.max()) if n > 0 else 0
        m4, strides = _mask_operand(mask, n, h, int(max_q_len), max_keys, dev)
        st = _lib.load().nia_prefill_masked(
            out.data_ptr(), out.stride(0), out.stride(1),
            q.data_ptr(), q.stride(0), q.stride(1),
            k.data_ptr(), k.stride(0), k.stride(1),
            v.data_ptr(), v.stride(0), v.stride(1),
            qs.data_ptr(), ql.data_ptr(), ks.data_ptr(), kl.data_ptr(),
            n, int(max_q_len), h, hkv, d, _default_scale(d, scale), int(causal), dt,
            m4.data_ptr(), *strides, _stream(dev),
        )
        _lib.check("nia_prefill_masked", st)
        return out
    lib = _lib.calls()
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


def _mask_operand(mask: torch.Tensor, num_seqs: int, num_heads: int, max_rows: int,
                  max_keys: int, device):
    """A 4-D additive mask [S or 1, H or 1, rows, keys] as the fp32 operand of
    nia_prefill_masked: 16-byte aligned, last dimension contiguous and every stride a
    multiple of four elements (a copy with the key dimension padded to a multiple of four
    when the given tensor is not); returns it and its (sequence, head, row) strides, 0
    for broadcast dimensions.  The kernels read rows below ``max_rows`` (the launch's
    longest query run) and keys below each sequence's key length (at most ``max_keys``),
    so a mask must cover them: a row or key dimension of size 1 broadcasts, and one that
    is shorter raises ValueError here instead of reading past the tensor."""
    if mask.dim() != 4:
        raise ValueError(f"mask must be 4-D [sequences, heads, rows, keys], got {tuple(mask.shape)}")
    if mask.shape[0] not in (1, num_seqs) or mask.shape[1] not in (1, num_heads):
        raise ValueError(f"mask of shape {tuple(mask.shape)} for {num_seqs} sequences and "
                         f"{num_heads} heads")
    if mask.shape[2] != 1 and mask.shape[2] < max_rows:
        raise ValueError(f"mask of shape {tuple(mask.shape)} has fewer rows than the "
                         f"{max_rows} queries of the longest sequence")
    if mask.shape[3] != 1 and mask.shape[3] < max_keys:
        raise ValueError(f"mask of shape {tuple(mask.shape)} has fewer keys than the "
                         f"{max_keys} of the longest sequence")
    if mask.shape[3] == 1 and max_keys > 1:
        mask = mask.expand(*mask.shape[:3], max_keys)  # the kernels read keys as a row
    m = mask.to(device=device, dtype=torch.float32)
    st = m.stride()
    ok = (m.stride(3) == 1 or m.shape[3] == 1) and m.data_ptr() % 16 == 0 and all(
        (st[i] % 4 == 0 or m.shape[i] == 1) for i in range(3))
    if not ok:
        keys = m.shape[3]
        padded = torch.zeros(*m.shape[:3], -(-keys // 4) * 4, dtype=torch.float32,
                             device=device)
        padded[..., :keys] = m
        m = padded
    strides = tuple(0 if m.shape[i] == 1 else m.stride(i) for i in range(3))
    return m, strides


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
    sizes the launch grid.  When it is omitted it is computed from cu_seqlens_q:
    on the host for a CPU tensor, else read back from the device once per
    cu_seqlens tensor (the blocks of a vision tower share one, see TensorMemo).
    cu_seqlens on the CPU are copied to q's device.
    """
    if cu_seqlens_k is None:
        cu_seqlens_k = cu_seqlens_q
    if max_seqlen_q is None:
        max_seqlen_q = _MAX_SEQLEN.get(cu_seqlens_q, "max")
        if max_seqlen_q is None:
            lens = cu_seqlens_q[1:] - cu_seqlens_q[:-1]
            max_seqlen_q = int(lens.max().item()) if lens.numel() else 0
            _MAX_SEQLEN.put(cu_seqlens_q, "max", max_seqlen_q)
    sq, lq = _starts_and_lengths(cu_seqlens_q, q.device)
    sk, lk = (sq, lq) if cu_seqlens_k is cu_seqlens_q else \
        _starts_and_lengths(cu_seqlens_k, q.device)
    return prefill(q, k, v, sq, lq, sk, lk, max_seqlen_q,
                   CAUSAL_TOP_LEFT if causal else CAUSAL_NONE, scale, out)


def _starts_and_lengths(cu: torch.Tensor, device) -> Tuple[torch.Tensor, torch.Tensor]:
    """int32 chunk starts and lengths on ``device`` from cumulative lengths, derived once
    per cu_seqlens tensor."""
    key = ("starts", device)
    got = _MAX_SEQLEN.get(cu, key)
    if got is None:
        c = cu.to(device=device, dtype=torch.int32)
        got = (c[:-1], c[1:] - c[:-1])
        _MAX_SEQLEN.put(cu, key, got)
    return got


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
    lib = _lib.calls()
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


class _QkPlan:
    """What qk_norm_rope_kv_write validated and derived for one argument signature."""

    __slots__ = ("n", "h", "hkv", "d", "q_tok", "q_head", "k_tok", "k_head", "v_tok",
                 "v_head", "v_copy", "num_axes", "sec0", "sec1", "pos_copy", "inv_copy", "w_copy",
                 "slot_copy", "write", "fp8", "bs", "nb", "dt", "eps")


_QK_PLANS: dict = {}


def _qk_plan(q, k, v, q_norm_weight, k_norm_weight, eps, positions, inv_freq, mrope_section,
             k_cache, v_cache, slot_mapping, k_scale, v_scale) -> _QkPlan:
    """Full validation of a qk_norm_rope_kv_write call (raises ValueError on a bad one)."""
    _require_gpu(q, k, v, positions, inv_freq)
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
    try:  # v is only read: one that is not viewable is copied for each call
        v2 = v.view(n, v.shape[-2], d)
        v_copy = False
    except RuntimeError:
        v2 = v.reshape(n, v.shape[-2], d)
        v_copy = True
    for name, t in (("q", q2), ("k", k2), ("v", v2)):
        _last_contig(name, t)
    pl = _QkPlan()
    if mrope_section is None:
        if positions.shape != lead:
            raise ValueError(f"positions must have shape {tuple(lead)}")
        pl.num_axes, pl.sec0, pl.sec1 = 1, 0, 0
    else:
        if positions.shape != (3, *lead):
            raise ValueError(f"mRoPE positions must have shape (3, {tuple(lead)})")
        pl.num_axes, pl.sec0, pl.sec1 = 3, int(mrope_section[0]), int(mrope_section[1])
    pl.pos_copy = positions.dtype != torch.int64 or not positions.is_contiguous()
    if not inv_freq.is_floating_point() or inv_freq.numel() != d // 2:
        raise ValueError(f"inv_freq must be a ({d // 2},) floating-point table")
    # A module cast to the model dtype holds a rounded table; the products
    # position * inv_freq are still formed in fp32 from those rounded values.
    pl.inv_copy = inv_freq.dtype != torch.float32 or not inv_freq.is_contiguous()
    pl.w_copy = False
    if q_norm_weight is not None:
        if q_norm_weight.shape != (d,) or k_norm_weight.shape != (d,) or \
                q_norm_weight.dtype != q.dtype or k_norm_weight.dtype != q.dtype:
            raise ValueError(f"norm weights must be ({d},) in the model dtype")
        if q_norm_weight.get_device() != q.get_device() or \
                k_norm_weight.get_device() != q.get_device():
            raise ValueError("norm weights must be on q's device")
        pl.w_copy = not (q_norm_weight.is_contiguous() and k_norm_weight.is_contiguous())
    pl.write, pl.fp8, pl.bs, pl.nb, pl.slot_copy = False, False, 1, 0, False
    if k_cache is not None:
        if v_cache is None or slot_mapping is None:
            raise ValueError("a cache write needs v_cache and slot_mapping")
        _require_gpu(q, k_cache, v_cache, slot_mapping)
        if k_cache.dim() != 4 or v_cache.shape != k_cache.shape or \
                k_cache.shape[1] != k2.shape[1] or k_cache.shape[3] != d:
            raise ValueError("k_cache/v_cache must be [num_blocks, H_kv, block_size, D]")
        if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
            raise ValueError("k_cache/v_cache layer slices must be contiguous")
        pl.fp8 = is_fp8_cache(k_cache)
        if pl.fp8:
            if v_cache.dtype != k_cache.dtype:
                raise ValueError("k_cache and v_cache must share one dtype")
            _fp8_scales(k_cache, k_scale, v_scale)
        elif k_cache.dtype != q.dtype or v_cache.dtype != q.dtype:
            raise ValueError("caches must share the model dtype")
        if slot_mapping.dtype != torch.int64 or slot_mapping.numel() != n:
            raise ValueError(f"slot_mapping must be int64 with {n} entries")
        pl.slot_copy = not slot_mapping.is_contiguous()
        pl.write, pl.nb, pl.bs = True, k_cache.shape[0], k_cache.shape[2]
    pl.n, pl.h, pl.hkv, pl.d, pl.dt, pl.eps = n, q2.shape[1], k2.shape[1], d, dt, float(eps)
    pl.q_tok, pl.q_head = q2.stride(0), q2.stride(1)
    pl.k_tok, pl.k_head = k2.stride(0), k2.stride(1)
    pl.v_tok, pl.v_head = v2.stride(0), v2.stride(1)
    pl.v_copy = v_copy
    return pl


def _inv_freq_f32(inv_freq: torch.Tensor) -> torch.Tensor:
    """The RoPE table as contiguous fp32, converted once per table: a module cast to the
    model dtype holds a rounded table, which every layer of every step passes."""
    t = _INV_FREQ_F32.get(inv_freq, "f32")
    if t is None:
        t = inv_freq.to(torch.float32).contiguous()
        _INV_FREQ_F32.put(inv_freq, "f32", t)
    return t


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
    A call is validated in full the first time its arguments' shapes, strides, dtypes and
    devices are seen; later calls with the same signature reuse that result.
    """
    nw = q_norm_weight is not None
    sig = (q.shape, q.stride(), q.dtype, q.get_device(), k.shape, k.stride(), k.dtype,
           k.get_device(), v.shape, v.stride(), v.dtype, v.get_device(),
           (q_norm_weight.shape, q_norm_weight.stride(), q_norm_weight.dtype,
            q_norm_weight.get_device()) if nw else None,
           (k_norm_weight.shape, k_norm_weight.stride(), k_norm_weight.dtype,
            k_norm_weight.get_device()) if k_norm_weight is not None else None,
           eps, positions.shape, positions.stride(), positions.dtype, positions.get_device(),
           inv_freq.shape, inv_freq.stride(), inv_freq.dtype, inv_freq.get_device(),
           mrope_section,
           (k_cache.shape, k_cache.stride(), k_cache.dtype, k_cache.get_device())
           if k_cache is not None else None,
           (v_cache.shape, v_cache.stride(), v_cache.dtype, v_cache.get_device())
           if v_cache is not None else None,
           (slot_mapping.shape, slot_mapping.stride(), slot_mapping.dtype,
            slot_mapping.get_device()) if slot_mapping is not None else None,
           (k_scale.shape, k_scale.stride(), k_scale.dtype, k_scale.get_device())
           if k_scale is not None else None,
           (v_scale.shape, v_scale.stride(), v_scale.dtype, v_scale.get_device())
           if v_scale is not None else None)
    pl = _QK_PLANS.get(sig)
    if pl is None:
        pl = _qk_plan(q, k, v, q_norm_weight, k_norm_weight, eps, positions, inv_freq,
                      mrope_section, k_cache, v_cache, slot_mapping, k_scale, v_scale)
        if len(_QK_PLANS) >= _PLAN_CACHE_MAX:
            _QK_PLANS.clear()
        _QK_PLANS[sig] = pl
    pos = positions.to(torch.int64).contiguous() if pl.pos_copy else positions
    inv = _inv_freq_f32(inv_freq) if pl.inv_copy else inv_freq
    qw, kw = q_norm_weight, k_norm_weight
    if pl.w_copy:
        qw, kw = qw.contiguous(), kw.contiguous()
    if pl.v_copy:
        v = v.reshape(pl.n, pl.hkv, pl.d)
    kc_ptr = vc_ptr = sl_ptr = None
    if pl.write:
        slots = slot_mapping.contiguous() if pl.slot_copy else slot_mapping
        kc_ptr, vc_ptr, sl_ptr = k_cache.data_ptr(), v_cache.data_ptr(), slots.data_ptr()
    lib = _lib.calls()
    args = (q.data_ptr(), pl.q_tok, pl.q_head, k.data_ptr(), pl.k_tok, pl.k_head,
            v.data_ptr(), pl.v_tok, pl.v_head,
            qw.data_ptr() if nw else None, kw.data_ptr() if nw else None,
            pl.eps, pos.data_ptr(), pl.n, pl.num_axes, inv.data_ptr(), pl.sec0, pl.sec1,
            kc_ptr, vc_ptr)
    tail = (sl_ptr, pl.n, pl.h, pl.hkv, pl.d, pl.bs, pl.nb, pl.dt,
            _raw_stream(q.get_device()))
    if pl.fp8:
        st = lib.nia_qk_norm_rope_kv_write_fp8(*args, k_scale.data_ptr(), v_scale.data_ptr(),
                                               *tail)
        if st:
            _lib.check("nia_qk_norm_rope_kv_write_fp8", st)
        return
    st = lib.nia_qk_norm_rope_kv_write(*args, *tail)
    if st:
        _lib.check("nia_qk_norm_rope_kv_write", st)
