"""Inputs whose attention logits reach tens of nats (test helpers).

Every kernel keeps a running maximum per row and raises it lazily: only when a new
block or tile of keys exceeds it by more than 2^8 (in log2 units) are the running
sum and output rescaled.  N(0, 1) inputs never get there, so these helpers build
queries and keys along a shared direction u (one per sequence and KV head):

    q = alpha * u + 0.5 * n,    k_t = lam(t) * u + m_t      (n, m ~ N(0, 1))

so that the logit of key t is about scale * alpha * lam(t) (with alpha = 12 and
D = 128 that is lam(t) nats), plus O(1) noise.  ``lam`` profiles:

  ramp      rises by ~0.4 nats per key up to ``top`` nats, then stays there: every
            later block or tile raises the running max by more than 2^8;
  late      zero, except two keys: one at a third of the context (top - 1 nats) and
            one near its end (top nats), whose values the output then mixes;
  fall      starts at ``top`` and falls by ~0.4 nats per key (exp underflow);
  scaled    no direction: q and every key multiplied by 4 (logits ~N(0, 16^2)).
"""
from __future__ import annotations

import math
from typing import List

import torch

ALPHA = 12.0


def lam_profile(n: int, mode: str, top: float, device) -> torch.Tensor:
    """lam(t) for t < n (float32, on ``device``); see the module docstring."""
    t = torch.arange(n, device=device, dtype=torch.float32)
    if mode == "ramp":
        return torch.clamp(t * 0.4, max=top)
    if mode == "fall":
        return top - t * 0.4
    if mode == "late":
        lam = torch.zeros(n, device=device)
        if n >= 3:
            lam[n // 3] = top - 1.0
            lam[n - 2] = top
        return lam
    raise ValueError(mode)


def directions(count: int, d: int, seed: int, device) -> torch.Tensor:
    """``count`` random unit vectors of length d (float32)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    u = torch.randn(count, d, generator=g)
    return (u / u.norm(dim=1, keepdim=True)).to(device)


def lam_scale(d: int) -> float:
    """Factor that turns lam (in nats) into the key component along u for head dim d."""
    return math.sqrt(d) / ALPHA


def shape_paged(kc: torch.Tensor, tables: List[List[int]], lens: List[int], u: torch.Tensor,
                mode: str, top: float) -> None:
    """Add lam(t) * u[i, hk] to key t of sequence i in a paged cache [NB, H_kv, BS, D]
    (block tables[i][t // BS], slot t % BS), for t < lens[i]."""
    d = kc.shape[3]
    bs = kc.shape[2]
    dev = kc.device
    for i, L in enumerate(lens):
        if L <= 0:
            continue
        lam = lam_profile(L, mode, top, dev) * lam_scale(d)
        ids = torch.tensor(tables[i], device=dev, dtype=torch.long)
        t = torch.arange(L, device=dev)
        blk, slot = ids[t // bs], t % bs
        rows = kc[blk, :, slot, :].float() + lam.view(L, 1, 1) * u[i].unsqueeze(0)
        kc[blk, :, slot, :] = rows.to(kc.dtype)


def shaped_queries(q: torch.Tensor, u: torch.Tensor, seed: int) -> torch.Tensor:
    """alpha * u (per KV head, repeated over its query heads) + 0.5 * N(0, 1), shaped
    and typed like q (rows, H, D); u is (rows, H_kv, D)."""
    h = q.shape[1]
    g = h // u.shape[1]
    gen = torch.Generator(device="cpu").manual_seed(seed)
    noise = (0.5 * torch.randn(q.shape, generator=gen)).to(q.device)
    return (ALPHA * u.repeat_interleave(g, dim=1) + noise).to(q.dtype)


def shape_decode(c, mode: str, top: float = 100.0, seed: int = 0, layer: int = 0) -> None:
    """Rewrite a workloads.DecodeCase in place (q, the cached keys of every sequence
    and its new key) so that its logits follow ``mode``."""
    b, h, d = c.q.shape
    hkv = c.num_kv_heads
    dev = c.q.device
    if mode == "scaled":
        c.q.mul_(4)
        c.k_new.mul_(4)
        c.k_cache[layer].mul_(4)
        return
    u = directions(b * hkv, d, seed, dev).view(b, hkv, d)
    c.q.copy_(shaped_queries(c.q, u, seed + 1))
    shape_paged(c.k_cache[layer], c.tables_list, c.lens, u, mode, top)
    # the new token (position L - 1) is written by the step from k_new
    for i, L in enumerate(c.lens):
        if L > 0:
            lam = float(lam_profile(L, mode, top, dev)[L - 1]) * lam_scale(d)
            c.k_new[i, 0] = (c.k_new[i, 0].float() + lam * u[i]).to(c.k_new.dtype)


def shape_chunked(c, mode: str, top: float = 100.0, seed: int = 0) -> None:
    """Rewrite a workloads.ChunkedCase in place: the chunk queries and every cached key."""
    n = len(c.prior)
    h, d = c.q.shape[1], c.q.shape[2]
    hkv = c.k_cache.shape[1]
    dev = c.q.device
    if mode == "scaled":
        c.q.mul_(4)
        c.k_cache.mul_(4)
        return
    u = directions(n * hkv, d, seed, dev).view(n, hkv, d)
    rows = c.q.view(n, c.chunk, h, d)
    for s in range(n):
        rows[s] = shaped_queries(rows[s], u[s].unsqueeze(0).expand(c.chunk, hkv, d), seed + 1 + s)
    shape_paged(c.k_cache, c.tables_list, [p + c.chunk for p in c.prior], u, mode, top)


def shape_rows(q: torch.Tensor, k: torch.Tensor, q_starts: List[int], q_lens: List[int],
               k_starts: List[int], k_lens: List[int], mode: str, top: float = 100.0,
               seed: int = 0) -> None:
    """Rewrite token-major q (T, H, D) and k (T, H_kv, D) in place, sequence by
    sequence, so that each row's logits over its keys follow ``mode`` (key t of a
    sequence gets lam(t))."""
    d = q.shape[2]
    hkv = k.shape[1]
    dev = q.device
    if mode == "scaled":
        q.mul_(4)
        k.mul_(4)
        return
    n = len(q_starts)
    u = directions(n * hkv, d, seed, dev).view(n, hkv, d)
    for s in range(n):
        qs, ql, ks, kl = q_starts[s], q_lens[s], k_starts[s], k_lens[s]
        if ql > 0:
            q[qs:qs + ql] = shaped_queries(q[qs:qs + ql], u[s].unsqueeze(0).expand(ql, hkv, d),
                                           seed + 1 + s)
        if kl > 0:
            lam = lam_profile(kl, mode, top, dev) * lam_scale(d)
            k[ks:ks + kl] = (k[ks:ks + kl].float() + lam.view(kl, 1, 1) * u[s].unsqueeze(0)
                             ).to(k.dtype)


def max_logit(q: torch.Tensor, k: torch.Tensor, scale: float) -> float:
    """Largest |scale * q . k| over all pairs of two small (n, D) / (m, D) sets."""
    return float((q.double() @ k.double().T).abs().max() * scale)
