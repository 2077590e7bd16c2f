"""Seeded synthetic inputs for the attention workloads (bench and tests).

Every tensor is N(0, 1) from a seeded torch.Generator; lengths are integers
drawn uniformly on closed intervals; block tables are consecutive slices of a
seeded permutation of the whole block pool, so physical order is scattered; the
whole pool is filled with N(0, 1) so that a kernel reading past a context or
through a wrong table entry picks up visible garbage.

Workloads (head layouts of the models the engine serves):
  decode_small    4 sequences, 16/8 heads, D 128, contexts 17/64/200/511,
                  block size 16, 128-block pool, fp32 (the CPU-runnable case)
  decode_qwen3_8b 64 sequences, 32/8 heads, D 128, contexts U[512, 8192],
                  40,000-block pool, bf16
  decode_vl       32 sequences, 28/4 heads, D 128, contexts U[1024, 6144], bf16
  prefill_qwen3_8b 8 packed sequences U[256, 4096], 32/8 heads, D 128, bf16
  chunked_qwen3_8b 8 chunks of 512 queries on top of U[0, 8192] cached tokens
  vision_vl       7528 patches of 4 images, 16 heads, D 80, full and window chunks
quantize_cache_fp8 turns a decode case's pool into the fp8 format (e4m3 codes plus
one scale per row) with the fp8 KV-write kernel; fp8_decode_bytes counts its bytes.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List, Optional, Tuple

import torch

VISION_GRIDS: List[Tuple[int, int, int]] = [(1, 28, 28), (1, 36, 52), (1, 64, 48), (1, 20, 90)]


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _randn(shape, dtype, device, seed) -> torch.Tensor:
    """N(0, 1) drawn in fp32 by a generator on ``device``, then cast."""
    return torch.randn(shape, generator=_gen(seed, device), device=device,
                       dtype=torch.float32).to(dtype)


def uniform_lengths(n: int, lo: int, hi: int, seed: int) -> List[int]:
    g = _gen(seed, "cpu")
    return torch.randint(lo, hi + 1, (n,), generator=g).tolist()


@dataclass
class DecodeCase:
    """One decode step: write the new token of every sequence, then attend."""

    q: torch.Tensor            # (B, H, D)
    k_new: torch.Tensor        # (B, 1, H_kv, D)
    v_new: torch.Tensor
    k_cache: torch.Tensor      # [layers, NB, H_kv, BS, D]
    v_cache: torch.Tensor
    block_tables: torch.Tensor  # (B, max_blocks) int32, zero-padded
    context_lens: torch.Tensor  # (B,) int64, includes the new token
    slot_mapping: torch.Tensor  # (B, 1) int64
    lens: List[int]
    block_size: int
    name: str = ""
    tables_list: List[List[int]] = field(default_factory=list)

    @property
    def batch(self) -> int:
        return self.q.shape[0]

    @property
    def num_heads(self) -> int:
        return self.q.shape[1]

    @property
    def num_kv_heads(self) -> int:
        return self.k_cache.shape[2]

    @property
    def head_dim(self) -> int:
        return self.q.shape[2]

    def kv_bytes(self) -> int:
        es = self.q.element_size()
        return sum(self.lens) * self.num_kv_heads * self.head_dim * es * 2

    def decode_bytes(self) -> int:
        """Algorithmic HBM bytes of one decode launch: K+V, q+out, tables, lens."""
        es = self.q.element_size()
        blocks = sum(math.ceil(L / self.block_size) for L in self.lens)
        return (self.kv_bytes() + 2 * self.batch * self.num_heads * self.head_dim * es
                + 4 * blocks + 8 * self.batch)

    def write_bytes(self) -> int:
        """Algorithmic bytes of the KV write: read and write K and V, plus slots."""
        es = self.q.element_size()
        return 4 * self.batch * self.num_kv_heads * self.head_dim * es + 8 * self.batch


@dataclass
class Fp8Cache:
    """A decode case's cache pool in the fp8 format (e4m3 codes, one scale per row)."""

    k_cache: torch.Tensor  # [layers, NB, H_kv, BS, D] uint8
    v_cache: torch.Tensor
    k_scale: torch.Tensor  # [layers, NB, H_kv, BS] float32
    v_scale: torch.Tensor


def quantize_cache_fp8(c: DecodeCase) -> Fp8Cache:
    """Every row of the case's pool written into fp8 caches by the fp8 KV-write kernel."""
    from . import ops

    layers, nb, hkv, bs, d = c.k_cache.shape
    dev = c.k_cache.device
    out = Fp8Cache(torch.empty((layers, nb, hkv, bs, d), dtype=torch.uint8, device=dev),
                   torch.empty((layers, nb, hkv, bs, d), dtype=torch.uint8, device=dev),
                   torch.zeros((layers, nb, hkv, bs), dtype=torch.float32, device=dev),
                   torch.zeros((layers, nb, hkv, bs), dtype=torch.float32, device=dev))
    slots = torch.arange(nb * bs, dtype=torch.int64, device=dev)
    for layer in range(layers):
        k_rows = c.k_cache[layer].transpose(1, 2).reshape(nb * bs, hkv, d)
        v_rows = c.v_cache[layer].transpose(1, 2).reshape(nb * bs, hkv, d)
        ops.kv_write(k_rows, v_rows, out.k_cache[layer], out.v_cache[layer], slots,
                     out.k_scale[layer], out.v_scale[layer])
        del k_rows, v_rows
    return out


def fp8_decode_bytes(c: DecodeCase) -> int:
    """Algorithmic HBM bytes of one decode launch over fp8 caches: K+V codes and row
    scales, bf16 q + out, tables, lens."""
    blocks = sum(math.ceil(L / c.block_size) for L in c.lens)
    return (sum(c.lens) * c.num_kv_heads * (c.head_dim + 4) * 2
            + 2 * c.batch * c.num_heads * c.head_dim * 2 + 4 * blocks + 8 * c.batch)


def make_decode(batch: int, num_heads: int, num_kv_heads: int, head_dim: int,
                lens: List[int], pool_blocks: int, block_size: int, dtype, device,
                seed: int, layers: int = 1, max_blocks: Optional[int] = None,
                name: str = "") -> DecodeCase:
    nblk = [math.ceil(L / block_size) for L in lens]
    if sum(nblk) > pool_blocks:
        raise ValueError("block pool too small for the drawn lengths")
    perm = torch.randperm(pool_blocks, generator=_gen(seed + 1, "cpu")).tolist()
    mb = max_blocks if max_blocks is not None else max(nblk)
    tables = torch.zeros((batch, mb), dtype=torch.int32)
    tl: List[List[int]] = []
    off = 0
    for i, n in enumerate(nblk):
        ids = perm[off:off + n]
        off += n
        tables[i, :n] = torch.tensor(ids, dtype=torch.int32)
        tl.append(ids)
    slots = torch.tensor([[tl[i][(L - 1) // block_size] * block_size + (L - 1) % block_size]
                          for i, L in enumerate(lens)], dtype=torch.int64)
    shape = (layers, pool_blocks, num_kv_heads, block_size, head_dim)
    return DecodeCase(
        q=_randn((batch, num_heads, head_dim), dtype, device, seed + 2),
        k_new=_randn((batch, 1, num_kv_heads, head_dim), dtype, device, seed + 3),
        v_new=_randn((batch, 1, num_kv_heads, head_dim), dtype, device, seed + 4),
        k_cache=_randn(shape, dtype, device, seed + 5),
        v_cache=_randn(shape, dtype, device, seed + 6),
        block_tables=tables.to(device),
        context_lens=torch.tensor(lens, dtype=torch.int64, device=device),
        slot_mapping=slots.to(device),
        lens=list(lens),
        block_size=block_size,
        name=name,
        tables_list=tl,
    )


def decode_small(device="cpu", dtype=torch.float32, seed: int = 1001) -> DecodeCase:
    return make_decode(4, 16, 8, 128, [17, 64, 200, 511], 128, 16, dtype, device, seed,
                       name="decode_small")


def decode_qwen3_8b(device="cuda", dtype=torch.bfloat16, seed: int = 2002, layers: int = 1,
                    batch: int = 64) -> DecodeCase:
    lens = uniform_lengths(batch, 512, 8192, seed)
    return make_decode(batch, 32, 8, 128, lens, 40000, 16, dtype, device, seed, layers=layers,
                       max_blocks=8192 // 16, name="decode_qwen3_8b")


def decode_vl(device="cuda", dtype=torch.bfloat16, seed: int = 5005, layers: int = 1) -> DecodeCase:
    lens = uniform_lengths(32, 1024, 6144, seed)
    return make_decode(32, 28, 4, 128, lens, 16384, 16, dtype, device, seed, layers=layers,
                       max_blocks=6144 // 16, name="decode_vl")


@dataclass
class VarlenCase:
    q: torch.Tensor  # (T, H, D)
    k: torch.Tensor  # (T, H_kv, D)
    v: torch.Tensor
    cu_seqlens: torch.Tensor  # (n + 1,) int32
    lens: List[int]
    causal: bool
    name: str = ""

    def flops(self) -> int:
        h, d = self.q.shape[1], self.q.shape[2]
        if self.causal:
            pairs = sum(n * (n + 1) // 2 for n in self.lens)
        else:
            pairs = sum(n * n for n in self.lens)
        return 4 * h * d * pairs


def make_varlen(lens: List[int], num_heads: int, num_kv_heads: int, head_dim: int, dtype,
                device, seed: int, causal: bool, name: str = "") -> VarlenCase:
    t = sum(lens)
    cu = torch.tensor([0] + lens, dtype=torch.int64).cumsum(0).to(torch.int32)
    return VarlenCase(
        q=_randn((t, num_heads, head_dim), dtype, device, seed + 1),
        k=_randn((t, num_kv_heads, head_dim), dtype, device, seed + 2),
        v=_randn((t, num_kv_heads, head_dim), dtype, device, seed + 3),
        cu_seqlens=cu.to(device),
        lens=list(lens),
        causal=causal,
        name=name,
    )


def prefill_qwen3_8b(device="cuda", dtype=torch.bfloat16, seed: int = 3003) -> VarlenCase:
    lens = uniform_lengths(8, 256, 4096, seed)
    return make_varlen(lens, 32, 8, 128, dtype, device, seed, True, "prefill_qwen3_8b")


@dataclass
class ChunkedCase:
    q: torch.Tensor  # (n * C, H, D)
    k_cache: torch.Tensor  # [NB, H_kv, BS, D], already holding every sequence's keys
    v_cache: torch.Tensor
    block_tables: torch.Tensor  # (n, max_blocks) int32
    q_start: torch.Tensor  # (n,) int32
    q_len: torch.Tensor  # (n,) int32
    context_lens: torch.Tensor  # (n,) int64 = prior + chunk
    prior: List[int]
    chunk: int
    block_size: int
    name: str = ""
    tables_list: List[List[int]] = field(default_factory=list)

    def flops(self) -> int:
        h, d = self.q.shape[1], self.q.shape[2]
        c = self.chunk
        return 4 * h * d * sum(c * p + c * (c + 1) // 2 for p in self.prior)


def chunked_qwen3_8b(device="cuda", dtype=torch.bfloat16, seed: int = 3103, n: int = 8,
                     chunk: int = 512, prior: Optional[List[int]] = None,
                     num_heads: int = 32, num_kv_heads: int = 8,
                     block_size: int = 16) -> ChunkedCase:
    prior = uniform_lengths(n, 0, 8192, seed) if prior is None else list(prior)
    bs = block_size
    ctx = [p + chunk for p in prior]
    nblk = [math.ceil(c / bs) for c in ctx]
    pool = max(sum(nblk) + 64, (1024 * 16) // bs)
    perm = torch.randperm(pool, generator=_gen(seed + 1, "cpu")).tolist()
    mb = max(nblk)
    tables = torch.zeros((n, mb), dtype=torch.int32)
    tl, off = [], 0
    for i, nb in enumerate(nblk):
        tables[i, :nb] = torch.tensor(perm[off:off + nb], dtype=torch.int32)
        tl.append(perm[off:off + nb])
        off += nb
    shape = (pool, num_kv_heads, bs, 128)
    return ChunkedCase(
        q=_randn((n * chunk, num_heads, 128), dtype, device, seed + 2),
        k_cache=_randn(shape, dtype, device, seed + 3),
        v_cache=_randn(shape, dtype, device, seed + 4),
        block_tables=tables.to(device),
        q_start=(torch.arange(n, dtype=torch.int32) * chunk).to(device),
        q_len=torch.full((n,), chunk, dtype=torch.int32, device=device),
        context_lens=torch.tensor(ctx, dtype=torch.int64, device=device),
        prior=prior,
        chunk=chunk,
        block_size=bs,
        name="chunked_qwen3_8b",
        tables_list=tl,
    )


def vision_vl(device="cuda", dtype=torch.bfloat16, seed: int = 5105, window: bool = False
              ) -> VarlenCase:
    from .vision import full_cu_seqlens, window_index

    cu = window_index(VISION_GRIDS)[1] if window else full_cu_seqlens(VISION_GRIDS)
    lens = [int(b - a) for a, b in zip(cu[:-1], cu[1:])]
    return make_varlen(lens, 16, 16, 80, dtype, device, seed, False,
                       "vision_vl_window" if window else "vision_vl_full")
