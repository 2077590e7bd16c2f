"""Prefill / chunked-prefill / vision varlen kernels vs the float64 oracle.

Oracle: oracle.textbook.varlen / paged_prefill (softmax(q K^T / sqrt(D)) V
with an explicit visible-key bound per row: top-left causal as the reference's
triu, src/nano_inference/layers/attention.py:33-38; bottom-right for chunks on
top of a cached context; none for the vision tower, layers/vision.py:190-208).
At full workload sizes a fixed sample of query rows (first, last, tile edges
and random rows) is checked; each sampled row is computed exactly.
Bars: bf16 max-abs 2e-2 / mean-abs 2e-3.
"""
import math

import numpy as np
import pytest
import torch

from nano_inference_amd import ops, workloads
from oracle import textbook as tb
from tests.tolerances import assert_attn_close

pytestmark = pytest.mark.gpu

MODES = {ops.CAUSAL_NONE: "none", ops.CAUSAL_TOP_LEFT: "top_left",
         ops.CAUSAL_BOTTOM_RIGHT: "bottom_right"}


def sample_rows(n: int, k: int, seed: int) -> np.ndarray:
    edges = [0, 1, 31, 32, 63, 64, 127, 128, 129, n // 2, n - 2, n - 1]
    rng = np.random.default_rng(seed)
    extra = rng.integers(0, n, size=max(0, k - len(edges)))
    return np.unique(np.clip(np.concatenate([edges, extra]), 0, n - 1))


def check_varlen(out, c: workloads.VarlenCase, mode: str, rows_per_seq=None, what=""):
    q, k, v = (t.double().cpu().numpy() for t in (c.q, c.k, c.v))
    cu = c.cu_seqlens.cpu().numpy()
    starts, lens = cu[:-1], cu[1:] - cu[:-1]
    rows = None
    if rows_per_seq is not None:
        rows = {s: sample_rows(int(n), rows_per_seq, s) for s, n in enumerate(lens)}
    res = tb.varlen(q, k, v, starts, lens, starts, lens, 1.0 / math.sqrt(q.shape[2]), mode, rows)
    got, exp = [], []
    o = out.double().cpu().numpy()
    for s, (idx, ref) in res.items():
        got.append(o[starts[s] + idx])
        exp.append(ref)
    assert_attn_close(np.concatenate(got), np.concatenate(exp), c.q.dtype, what)


def test_causal_prefill_qwen3_8b():
    """8 packed sequences U[256, 4096], 32/8 heads, D 128 (sampled rows)."""
    c = workloads.prefill_qwen3_8b("cuda")
    out = ops.varlen_attention(c.q, c.k, c.v, c.cu_seqlens, causal=True)
    torch.cuda.synchronize()
    check_varlen(out, c, "top_left", rows_per_seq=160, what="prefill_qwen3_8b")


@pytest.mark.parametrize("head_dim", [64, 80, 96, 128])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("group", [1, 4])
def test_varlen_small_full(head_dim, causal, group):
    lens = [1, 2, 63, 64, 65, 127, 128, 129, 200, 300]
    c = workloads.make_varlen(lens, 2 * group, 2, head_dim, torch.bfloat16, "cuda",
                              seed=head_dim + 7 * group + causal, causal=causal)
    out = ops.varlen_attention(c.q, c.k, c.v, c.cu_seqlens, causal=causal)
    torch.cuda.synchronize()
    check_varlen(out, c, "top_left" if causal else "none", what=f"D={head_dim} G={group}")


@pytest.mark.parametrize("head_dim", [64, 80, 128])
@pytest.mark.parametrize("heads", [2, 16])
def test_short_unmasked_sequences_paired_heads(head_dim, heads):
    """Sequences of at most 64 rows, no mask, one query head per KV head: the kernel
    takes two heads per workgroup (every row checked, lengths 1 .. 64)."""
    lens = [1, 2, 15, 16, 17, 31, 32, 33, 47, 63, 64, 64, 5]
    c = workloads.make_varlen(lens, heads, heads, head_dim, torch.bfloat16, "cuda",
                              seed=300 + head_dim + heads, causal=False)
    out = ops.varlen_attention(c.q, c.k, c.v, c.cu_seqlens, causal=False)
    torch.cuda.synchronize()
    check_varlen(out, c, "none", what=f"paired heads D={head_dim} H={heads}")


def test_ranked_grid_ties_and_empty_sequences():
    """Non-causal calls issue the grid longest sequence first (a rank computed in every
    workgroup): equal lengths, empty sequences and several m-blocks per sequence, every
    row checked."""
    lens = [300, 0, 129, 300, 64, 0, 129, 1, 300, 257]
    c = workloads.make_varlen(lens, 8, 2, 128, torch.bfloat16, "cuda", seed=910, causal=False)
    out = ops.varlen_attention(c.q, c.k, c.v, c.cu_seqlens, causal=False)
    torch.cuda.synchronize()
    check_varlen(out, c, "none", what="ranked grid")


def test_more_sequences_than_the_ranking_takes():
    """301 sequences (the rank holds 256): the grid falls back to the m-block-major map."""
    g = torch.Generator().manual_seed(911)
    lens = [int(x) for x in torch.randint(1, 151, (301,), generator=g)]
    c = workloads.make_varlen(lens, 8, 2, 64, torch.bfloat16, "cuda", seed=912, causal=False)
    out = ops.varlen_attention(c.q, c.k, c.v, c.cu_seqlens, causal=False)
    torch.cuda.synchronize()
    check_varlen(out, c, "none", what="301 sequences")


def test_bottom_right_contiguous_chunks():
    """Contiguous K/V longer than the queries (bottom-right mask, ranked grid): query
    chunks of 1..200 rows on 0..700 earlier keys, and a chunk longer than its keys whose
    first rows see none (zeros)."""
    g = torch.Generator().manual_seed(913)
    ql = [int(x) for x in torch.randint(1, 201, (9,), generator=g)] + [5]
    kl = [q + int(x) for q, x in zip(ql[:-1], torch.randint(0, 701, (9,), generator=g))] + [2]
    h, hkv, d = 8, 2, 128
    tq, tk = sum(ql), sum(kl)
    q = torch.randn(tq, h, d, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(tk, hkv, d, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(tk, hkv, d, generator=g).to(torch.bfloat16).cuda()
    qs = torch.tensor([0] + ql[:-1]).cumsum(0).to(torch.int32).cuda()
    ks = torch.tensor([0] + kl[:-1]).cumsum(0).to(torch.int32).cuda()
    qlt = torch.tensor(ql, dtype=torch.int32).cuda()
    klt = torch.tensor(kl, dtype=torch.int32).cuda()
    out = ops.prefill(q, k, v, qs, qlt, ks, klt, max(ql), ops.CAUSAL_BOTTOM_RIGHT)
    torch.cuda.synchronize()
    res = tb.varlen(q.double().cpu().numpy(), k.double().cpu().numpy(),
                    v.double().cpu().numpy(), qs.cpu().numpy(), ql, ks.cpu().numpy(), kl,
                    1.0 / math.sqrt(d), "bottom_right")
    o = out.double().cpu().numpy()
    got = np.concatenate([o[int(qs[s]) + idx] for s, (idx, _) in res.items()])
    exp = np.concatenate([ref for _, (_, ref) in res.items()])
    assert_attn_close(got, exp, torch.bfloat16, "bottom-right contiguous")
    assert np.all(o[int(qs[-1]):int(qs[-1]) + 3] == 0)


def test_vision_full_attention_chunks():
    """7528 patches in 4 images, 16 heads, D 80, non-causal per image (sampled rows)."""
    c = workloads.vision_vl("cuda", window=False)
    out = ops.varlen_attention(c.q, c.k, c.v, c.cu_seqlens, causal=False)
    torch.cuda.synchronize()
    check_varlen(out, c, "none", rows_per_seq=200, what="vision full")


def test_vision_window_chunks():
    """135 windows of 8..64 patches, every row checked."""
    c = workloads.vision_vl("cuda", window=True)
    out = ops.varlen_attention(c.q, c.k, c.v, c.cu_seqlens, causal=False)
    torch.cuda.synchronize()
    check_varlen(out, c, "none", what="vision windows")


def test_padded_layout_rows_past_length_see_all_keys():
    """Reference padded (B, S_max) prefill: rows j >= len attend keys [0, len)."""
    b, smax, h, hkv, d = 3, 150, 4, 2, 128
    lens = [150, 97, 1]
    g = torch.Generator(device="cuda").manual_seed(21)
    q = torch.randn((b * smax, h, d), generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn((b * smax, hkv, d), generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn((b * smax, hkv, d), generator=g, device="cuda").to(torch.bfloat16)
    starts = torch.arange(b, dtype=torch.int32, device="cuda") * smax
    ql = torch.full((b,), smax, dtype=torch.int32, device="cuda")
    kl = torch.tensor(lens, dtype=torch.int32, device="cuda")
    out = ops.prefill(q, k, v, starts, ql, starts, kl, smax, ops.CAUSAL_TOP_LEFT)
    torch.cuda.synchronize()
    qn, kn, vn = (t.double().cpu().numpy() for t in (q, k, v))
    res = tb.varlen(qn, kn, vn, starts.cpu().numpy(), [smax] * b, starts.cpu().numpy(), lens,
                    1 / math.sqrt(d), "top_left")
    o = out.double().cpu().numpy()
    for s, (idx, ref) in res.items():
        assert_attn_close(o[s * smax + idx], ref, torch.bfloat16, f"padded seq {s}")


def _chunk_oracle(c: workloads.ChunkedCase, rows_per_seq):
    q = c.q.double().cpu().numpy()
    res = {}
    scale = 1 / math.sqrt(q.shape[2])
    hkv = c.k_cache.shape[1]
    g = q.shape[1] // hkv
    for s in range(len(c.prior)):
        L = c.prior[s] + c.chunk
        ids = torch.tensor(c.tables_list[s], device=c.k_cache.device)
        kk = c.k_cache[ids].double().cpu().numpy().transpose(1, 0, 2, 3).reshape(hkv, -1, 128)[:, :L]
        vv = c.v_cache[ids].double().cpu().numpy().transpose(1, 0, 2, 3).reshape(hkv, -1, 128)[:, :L]
        idx = sample_rows(c.chunk, rows_per_seq, s) if rows_per_seq else np.arange(c.chunk)
        bnd = tb.causal_bounds(c.chunk, L, "bottom_right")[idx]
        o = np.zeros((len(idx), q.shape[1], 128))
        for hh in range(q.shape[1]):
            o[:, hh] = tb.attend(q[s * c.chunk + idx, hh], kk[hh // g], vv[hh // g], scale, bnd)
        res[s] = (idx, o)
    return res


def test_chunked_prefill_qwen3_8b():
    """512-query chunks on top of U[0, 8192] cached tokens, block size 16 (sampled rows)."""
    c = workloads.chunked_qwen3_8b("cuda")
    out = ops.prefill_paged(c.q, c.k_cache, c.v_cache, c.block_tables, c.q_start, c.q_len,
                            c.context_lens, c.chunk)
    torch.cuda.synchronize()
    o = out.double().cpu().numpy()
    for s, (idx, ref) in _chunk_oracle(c, 48).items():
        assert_attn_close(o[s * c.chunk + idx], ref, torch.bfloat16, f"chunk {s}")


def test_chunked_prefill_edges_full():
    """Prior lengths on block and tile edges, every row checked."""
    c = workloads.chunked_qwen3_8b("cuda", n=6, chunk=80, prior=[0, 1, 15, 16, 63, 200])
    out = ops.prefill_paged(c.q, c.k_cache, c.v_cache, c.block_tables, c.q_start, c.q_len,
                            c.context_lens, c.chunk)
    torch.cuda.synchronize()
    o = out.double().cpu().numpy()
    for s, (idx, ref) in _chunk_oracle(c, None).items():
        assert_attn_close(o[s * c.chunk + idx], ref, torch.bfloat16, f"chunk edge {s}")


@pytest.mark.parametrize("bs", [32, 64, 128, 256])
def test_chunked_prefill_block_sizes_full(bs):
    """Block sizes beyond 16: prior lengths on both sides of block edges and a chunk that
    crosses blocks, every row checked."""
    prior = [0, 1, bs - 1, bs, bs + 1, 3 * bs - 7]
    c = workloads.chunked_qwen3_8b("cuda", n=6, chunk=80, prior=prior, num_heads=8,
                                   num_kv_heads=2, block_size=bs)
    out = ops.prefill_paged(c.q, c.k_cache, c.v_cache, c.block_tables, c.q_start, c.q_len,
                            c.context_lens, c.chunk)
    torch.cuda.synchronize()
    o = out.double().cpu().numpy()
    for s, (idx, ref) in _chunk_oracle(c, None).items():
        assert_attn_close(o[s * c.chunk + idx], ref, torch.bfloat16, f"bs {bs} chunk {s}")


@pytest.mark.parametrize("bs,group", [(1, 4), (5, 4), (12, 4), (24, 7), (100, 2), (48, 4),
                                      (80, 2)])
def test_chunked_prefill_other_block_sizes_full(bs, group):
    """Block sizes that are not powers of two (the reference's block size is any positive
    integer, src/nano_inference/core/config.py:54): multiples of 16 (48, 80) on the DMA
    kernel, others of at least 2 on the register-staged kernel (both divide keys by the block
    size), block size 1 on the fp32-softmax kernel: prior lengths on both sides of block
    edges, every row checked."""
    prior = [0, 1, max(bs - 1, 0), bs, bs + 1, 3 * bs + 7]
    c = workloads.chunked_qwen3_8b("cuda", n=6, chunk=80, prior=prior, num_heads=2 * group,
                                   num_kv_heads=2, block_size=bs)
    out = ops.prefill_paged(c.q, c.k_cache, c.v_cache, c.block_tables, c.q_start, c.q_len,
                            c.context_lens, c.chunk)
    torch.cuda.synchronize()
    o = out.double().cpu().numpy()
    for s, (idx, ref) in _chunk_oracle(c, None).items():
        assert_attn_close(o[s * c.chunk + idx], ref, torch.bfloat16, f"bs {bs} chunk {s}")


def test_chunk_rows_equal_full_prefill_rows():
    """A chunk at positions P.. of a sequence equals those rows of the full causal prefill."""
    n, p_len, chunk, bs = 1, 700, 300, 16
    total = p_len + chunk
    g = torch.Generator(device="cuda").manual_seed(4)
    q = torch.randn((total, 8, 128), generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn((total, 2, 128), generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn((total, 2, 128), generator=g, device="cuda").to(torch.bfloat16)
    nblk = -(-total // bs)
    ids = torch.randperm(nblk + 9, generator=torch.Generator().manual_seed(2))[:nblk]
    kc = torch.zeros((nblk + 9, 2, bs, 128), dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    slots = (ids.repeat_interleave(bs)[:total] * bs + torch.arange(total) % bs).cuda()
    ops.kv_write(k, v, kc, vc, slots)
    bt = ids.to(torch.int32).view(1, -1).cuda()
    z = torch.zeros(1, dtype=torch.int32, device="cuda")
    out_c = ops.prefill_paged(q[p_len:].contiguous(), kc, vc, bt, z,
                              torch.tensor([chunk], dtype=torch.int32, device="cuda"),
                              torch.tensor([total], dtype=torch.int64, device="cuda"), chunk)
    tl = torch.tensor([total], dtype=torch.int32, device="cuda")
    out_f = ops.prefill(q, k, v, z, tl, z, tl, total, ops.CAUSAL_TOP_LEFT)
    torch.cuda.synchronize()
    assert_attn_close(out_c, out_f[p_len:].double().cpu().numpy(), torch.bfloat16,
                      "chunk vs full")


def test_causality_future_keys_do_not_change_past_rows():
    """Mirror of tests/unit/test_attention.py:16-33 on the kernel."""
    c = workloads.make_varlen([300], 4, 2, 128, torch.bfloat16, "cuda", 31, True)
    out1 = ops.varlen_attention(c.q, c.k, c.v, c.cu_seqlens, causal=True)
    k2, v2 = c.k.clone(), c.v.clone()
    k2[150:] = torch.randn_like(k2[150:].float()).to(torch.bfloat16)
    v2[150:] = torch.randn_like(v2[150:].float()).to(torch.bfloat16)
    out2 = ops.varlen_attention(c.q, k2, v2, c.cu_seqlens, causal=True)
    torch.cuda.synchronize()
    assert_attn_close(out1[:150], out2[:150].double().cpu().numpy(), torch.bfloat16, "causality")
