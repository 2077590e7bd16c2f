"""Float64 numpy attention with explicit visible-key bounds (oracle).

TEST INFRASTRUCTURE ONLY.

The reference's attention is softmax(q k^T / sqrt(D) + mask) v with fp32
softmax (src/nano_inference/layers/attention.py:12-50).  This module evaluates
the same mathematics in float64, row by row, with the mask expressed as a
number of visible keys per query row, so that causal (triu, :33-38), padding
(:321-326, :40-47) and paged-context bounds are one mechanism.  It shares no
code with the torch restatement in reference_attention.py; the two check each
other.  ``attend_bruteforce`` is the definition written as loops, for tiny
inputs.
"""
from __future__ import annotations

import math
from typing import Optional, Sequence

import numpy as np


def attend(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float,
           bounds: Optional[np.ndarray] = None) -> np.ndarray:
    """Rows of softmax(scale * q k^T) v over keys [0, bounds[i]).

    q: (n, D); k, v: (m, D); bounds: (n,) ints (None = all m keys).
    Rows with no visible key are 0 (the kernels' convention).
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    n, m = q.shape[0], k.shape[0]
    s = (q @ k.T) * scale
    if bounds is not None:
        cols = np.arange(m)[None, :]
        s = np.where(cols < np.asarray(bounds)[:, None], s, -np.inf)
    mx = s.max(axis=1, keepdims=True) if m else np.zeros((n, 1))
    safe = np.where(np.isfinite(mx), mx, 0.0)
    p = np.exp(s - safe)
    den = p.sum(axis=1, keepdims=True)
    out = np.zeros((n, v.shape[1]))
    ok = den[:, 0] > 0
    out[ok] = (p[ok] @ v) / den[ok]
    return out


def attend_bruteforce(q: Sequence[Sequence[float]], k, v, scale: float,
                      bounds: Optional[Sequence[int]] = None):
    """The same definition as plain Python loops (tiny inputs only)."""
    out = []
    for i, qi in enumerate(q):
        nb = len(k) if bounds is None else bounds[i]
        if nb <= 0:
            out.append([0.0] * len(v[0]))
            continue
        sc = [scale * sum(a * b for a, b in zip(qi, k[j])) for j in range(nb)]
        mx = max(sc)
        w = [math.exp(x - mx) for x in sc]
        tot = sum(w)
        out.append([sum(w[j] * v[j][c] for j in range(nb)) / tot for c in range(len(v[0]))])
    return out


def causal_bounds(q_len: int, k_len: int, mode: str) -> np.ndarray:
    """Visible-key counts per query row.

    mode 'none': k_len for every row; 'top_left': min(j + 1, k_len) (the
    reference's triu when S_q == S_k, extended to padded rows); 'bottom_right':
    k_len - q_len + j + 1 clipped to [0, k_len] (a query chunk at the end of its
    context, as chunked prefill needs).
    """
    j = np.arange(q_len)
    if mode == "none":
        b = np.full(q_len, k_len)
    elif mode == "top_left":
        b = np.minimum(j + 1, k_len)
    elif mode == "bottom_right":
        b = k_len - q_len + j + 1
    else:
        raise ValueError(mode)
    return np.clip(b, 0, k_len)


def gather_paged(cache: np.ndarray, block_table: np.ndarray, length: int, kv_head: int) -> np.ndarray:
    """Keys [0, length) of one sequence and KV head from a [NB, H_kv, BS, D] cache."""
    bs = cache.shape[2]
    t = np.arange(length)
    return cache[block_table[t // bs], kv_head, t % bs, :]


def paged_decode(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                 block_tables: np.ndarray, context_lens: np.ndarray, scale: float,
                 seqs: Optional[Sequence[int]] = None) -> np.ndarray:
    """q: (B, H, D) -> (B, H, D) float64 (rows of unlisted seqs left 0).

    Query head h reads KV head h // (H / H_kv) (repeat_interleave,
    src/nano_inference/layers/attention.py:310-314).
    """
    b, h, d = q.shape
    hkv = k_cache.shape[1]
    g = h // hkv
    out = np.zeros((b, h, d))
    for i in (range(b) if seqs is None else seqs):
        L = int(context_lens[i])
        for hk in range(hkv):
            kk = gather_paged(k_cache, block_tables[i], L, hk)
            vv = gather_paged(v_cache, block_tables[i], L, hk)
            out[i, hk * g:(hk + 1) * g] = attend(q[i, hk * g:(hk + 1) * g], kk, vv, scale)
    return out


def varlen(q: np.ndarray, k: np.ndarray, v: np.ndarray, q_start, q_len, k_start, k_len,
           scale: float, mode: str, rows: Optional[dict] = None) -> dict:
    """Per-sequence varlen attention on token-major (T, H, D) arrays.

    Returns {seq: (row_indices, out (n_rows, H, D))}; ``rows`` optionally picks a
    subset of query rows per sequence (each row is computed exactly).
    """
    h = q.shape[1]
    hkv = k.shape[1]
    g = h // hkv
    res = {}
    for s in range(len(q_start)):
        ql, kl = int(q_len[s]), int(k_len[s])
        idx = np.arange(ql) if rows is None or s not in rows else np.asarray(rows[s])
        bnd = causal_bounds(ql, kl, mode)[idx]
        qs, ks = int(q_start[s]), int(k_start[s])
        o = np.zeros((len(idx), h, q.shape[2]))
        for hh in range(h):
            hk = hh // g
            o[:, hh] = attend(q[qs + idx, hh], k[ks:ks + kl, hk], v[ks:ks + kl, hk], scale, bnd)
        res[s] = (idx, o)
    return res


def paged_prefill(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                  block_tables: np.ndarray, q_start, q_len, context_lens, scale: float,
                  mode: str = "bottom_right", rows: Optional[dict] = None) -> dict:
    """Query chunks against paged keys [0, context_len) (bottom-right causal)."""
    h = q.shape[1]
    hkv = k_cache.shape[1]
    g = h // hkv
    res = {}
    for s in range(len(q_start)):
        ql, L = int(q_len[s]), int(context_lens[s])
        idx = np.arange(ql) if rows is None or s not in rows else np.asarray(rows[s])
        bnd = causal_bounds(ql, L, mode)[idx]
        qs = int(q_start[s])
        o = np.zeros((len(idx), h, q.shape[2]))
        for hk in range(hkv):
            kk = gather_paged(k_cache, block_tables[s], L, hk)
            vv = gather_paged(v_cache, block_tables[s], L, hk)
            for hh in range(hk * g, (hk + 1) * g):
                o[:, hh] = attend(q[qs + idx, hh], kk, vv, scale, bnd)
        res[s] = (idx, o)
    return res
