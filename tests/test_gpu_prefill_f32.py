"""fp32 prefill (nia_prefill / nia_prefill_paged with NIA_DTYPE_F32) vs the float64 oracle.

The reference's shipped configuration runs float32 (configs/default.yaml:4), so every
S_q > 1 attention call of the fp32 model - the drop-in scaled_dot_product_attention
(src/nano_inference/layers/attention.py:12-50), the prefill branch (:281-284), chunked
prefill over the cache and the vision tower (src/nano_inference/layers/vision.py:
190-208) - runs the fp32 kernel.  Oracle: oracle.textbook in float64, every row.
Bar: max-abs 1e-5 (fp32), including logits of ~100 nats (tests/logit_inputs.py).
"""
import math

import numpy as np
import pytest
import torch

from nano_inference_amd import AttentionMetadata, PagedCausalSelfAttention, ops, workloads
from nano_inference_amd import scaled_dot_product_attention
from oracle import metadata as meta
from oracle import reference_attention as ref
from oracle import textbook as tb
from tests import logit_inputs as LI
from tests.tolerances import assert_attn_close

pytestmark = pytest.mark.gpu

F32 = torch.float32


def check(out, q, k, v, qs, ql, ks, kl, mode, what):
    res = tb.varlen(q.double().cpu().numpy(), k.double().cpu().numpy(), v.double().cpu().numpy(),
                    qs, ql, ks, kl, 1.0 / math.sqrt(q.shape[2]), mode)
    o = out.double().cpu().numpy()
    got = np.concatenate([o[int(qs[s]) + idx] for s, (idx, _) in res.items()])
    exp = np.concatenate([r for _, (_, r) in res.items()])
    assert_attn_close(got, exp, F32, what)


def test_causal_small_batch_layout():
    """16/8 heads, D 128, sequences of 17, 64, 200 and 511 tokens (the fp32 decode
    workload's lengths, as a causal prefill), every row."""
    lens = [17, 64, 200, 511]
    c = workloads.make_varlen(lens, 16, 8, 128, F32, "cuda", seed=1101, causal=True)
    out = ops.varlen_attention(c.q, c.k, c.v, c.cu_seqlens, causal=True)
    torch.cuda.synchronize()
    cu = c.cu_seqlens.tolist()
    check(out, c.q, c.k, c.v, cu[:-1], lens, cu[:-1], lens, "top_left", "fp32 causal, small batch")


@pytest.mark.parametrize("head_dim", [64, 80, 96, 128])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("group", [1, 4])
def test_varlen_full(head_dim, causal, group):
    lens = [1, 2, 15, 16, 17, 63, 64, 65, 129, 300]
    c = workloads.make_varlen(lens, 2 * group, 2, head_dim, F32, "cuda",
                              seed=1110 + head_dim + group + causal, causal=causal)
    out = ops.varlen_attention(c.q, c.k, c.v, c.cu_seqlens, causal=causal)
    torch.cuda.synchronize()
    cu = c.cu_seqlens.tolist()
    check(out, c.q, c.k, c.v, cu[:-1], lens, cu[:-1], lens, "top_left" if causal else "none",
          f"fp32 D={head_dim} G={group} causal={causal}")


def test_vision_window_and_full_d80():
    """The vision tower in fp32: D 80, non-causal, 16 heads, the 4-image grids' windows."""
    for window in (True, False):
        c = workloads.vision_vl("cuda", dtype=F32, window=window)
        out = ops.varlen_attention(c.q, c.k, c.v, c.cu_seqlens, causal=False)
        torch.cuda.synchronize()
        cu = c.cu_seqlens.tolist()
        if window:
            check(out, c.q, c.k, c.v, cu[:-1], c.lens, cu[:-1], c.lens, "none",
                  "fp32 vision windows")
        else:  # full attention: the first 300 rows of each image
            rows = [min(n, 300) for n in c.lens]
            check(out, c.q, c.k, c.v, cu[:-1], rows, cu[:-1], c.lens, "none", "fp32 vision full")


def test_bottom_right_and_padded_layouts():
    g = torch.Generator().manual_seed(1120)
    ql = [5, 64, 1, 130]
    kl = [5 + 300, 64 + 17, 1, 130]
    h, hkv, d = 8, 2, 128
    q = torch.randn(sum(ql), h, d, generator=g).cuda()
    k = torch.randn(sum(kl), hkv, d, generator=g).cuda()
    v = torch.randn(sum(kl), hkv, d, generator=g).cuda()
    qs = [0] + list(np.cumsum(ql)[:-1])
    ks = [0] + list(np.cumsum(kl)[:-1])
    i32 = dict(dtype=torch.int32, device="cuda")
    out = ops.prefill(q, k, v, torch.tensor(qs, **i32), torch.tensor(ql, **i32),
                      torch.tensor(ks, **i32), torch.tensor(kl, **i32), max(ql),
                      ops.CAUSAL_BOTTOM_RIGHT)
    torch.cuda.synchronize()
    check(out, q, k, v, qs, ql, ks, kl, "bottom_right", "fp32 bottom-right")
    # the reference's padded (B, S_max) batch: rows past a sequence's length see its keys
    smax, lens = 70, [70, 33]
    qp = torch.randn(2 * smax, h, d, generator=g).cuda()
    kp = torch.randn(2 * smax, hkv, d, generator=g).cuda()
    vp = torch.randn(2 * smax, hkv, d, generator=g).cuda()
    st = [0, smax]
    out = ops.prefill(qp, kp, vp, torch.tensor(st, **i32), torch.tensor([smax] * 2, **i32),
                      torch.tensor(st, **i32), torch.tensor(lens, **i32), smax,
                      ops.CAUSAL_TOP_LEFT)
    torch.cuda.synchronize()
    check(out, qp, kp, vp, st, [smax] * 2, st, lens, "top_left", "fp32 padded")


def _paged_case(prior, chunk, bs, h, hkv, d, seed, pool_extra=7):
    """Chunks of ``chunk`` queries after ``prior`` cached tokens, in a paged fp32 cache of
    block size ``bs`` (any value) with shuffled block ids."""
    g = torch.Generator().manual_seed(seed)
    ctx = [p + chunk for p in prior]
    nblk = [-(-c // bs) for c in ctx]
    pool = sum(nblk) + pool_extra
    perm = torch.randperm(pool, generator=g).tolist()
    mb = max(nblk)
    tables = torch.zeros((len(prior), mb), dtype=torch.int32)
    tl, off = [], 0
    for i, n in enumerate(nblk):
        tables[i, :n] = torch.tensor(perm[off:off + n], dtype=torch.int32)
        tl.append(perm[off:off + n])
        off += n
    kc = torch.randn(pool, hkv, bs, d, generator=g).cuda()
    vc = torch.randn(pool, hkv, bs, d, generator=g).cuda()
    q = torch.randn(len(prior) * chunk, h, d, generator=g).cuda()
    return q, kc, vc, tables.cuda(), tl, ctx


def _paged_oracle(q, kc, vc, tl, ctx, chunk):
    qn, kn, vn = q.double().cpu().numpy(), kc.double().cpu().numpy(), vc.double().cpu().numpy()
    n = len(ctx)
    res = tb.paged_prefill(qn, kn, vn, [np.asarray(t) for t in tl], [s * chunk for s in range(n)],
                           [chunk] * n, ctx, 1.0 / math.sqrt(q.shape[2]))
    return np.concatenate([r for _, (_, r) in res.items()])


@pytest.mark.parametrize("bs", [1, 8, 12, 16, 32, 64])
def test_chunked_prefill_block_sizes(bs):
    """Chunked prefill over an fp32 paged cache of block size 1 .. 64 (including a size
    that is not a power of two), chunks on block edges and after empty contexts."""
    prior, chunk = [0, 1, bs - 1 if bs > 1 else 2, 3 * bs, 200], 40
    q, kc, vc, bt, tl, ctx = _paged_case(prior, chunk, bs, 8, 2, 128, seed=1130 + bs)
    n = len(prior)
    i32 = dict(dtype=torch.int32, device="cuda")
    out = ops.prefill_paged(q, kc, vc, bt, torch.arange(n, **i32) * chunk,
                            torch.full((n,), chunk, **i32),
                            torch.tensor(ctx, dtype=torch.int64, device="cuda"), chunk)
    torch.cuda.synchronize()
    assert_attn_close(out, _paged_oracle(q, kc, vc, tl, ctx, chunk), F32, f"fp32 chunked bs={bs}")


@pytest.mark.parametrize("mode", ["ramp", "late", "fall", "scaled"])
def test_large_logits(mode):
    """Logits of ~100 nats: the scores are summed in fp64, so the fp32 bar holds."""
    lens = [1, 65, 300, 700]
    c = workloads.make_varlen(lens, 8, 2, 128, F32, "cuda", seed=1140, causal=True)
    cu = c.cu_seqlens.tolist()
    LI.shape_rows(c.q, c.k, cu[:-1], lens, cu[:-1], lens, mode, seed=71)
    out = ops.varlen_attention(c.q, c.k, c.v, c.cu_seqlens, causal=True)
    torch.cuda.synchronize()
    check(out, c.q, c.k, c.v, cu[:-1], lens, cu[:-1], lens, "top_left", f"fp32 causal {mode}")


def test_sdpa_free_function_fp32():
    """The drop-in scaled_dot_product_attention in fp32: causal (S_q == S_k), a prefix
    padding mask, and non-causal S_q != S_k (the reference then applies no triu)."""
    g = torch.Generator().manual_seed(1150)
    b, h, hkv, s, d = 2, 4, 2, 70, 64
    q = torch.randn(b, h, s, d, generator=g)
    k = torch.randn(b, hkv, s, d, generator=g)
    v = torch.randn(b, hkv, s, d, generator=g)
    lens = torch.tensor([70, 41])
    mask2d = torch.arange(s).unsqueeze(0) < lens.unsqueeze(1)
    add = ref.additive_mask(mask2d, torch.float64)
    out = scaled_dot_product_attention(q.cuda(), k.cuda(), v.cuda(), add.cuda(), is_causal=True)
    kr = k.double().repeat_interleave(h // hkv, dim=1)
    vr = v.double().repeat_interleave(h // hkv, dim=1)
    exp = ref.sdpa(q.double(), kr, vr, attention_mask=add, is_causal=True)
    assert_attn_close(out, exp, F32, "fp32 sdpa causal + mask")
    q1 = q[:, :, :9].contiguous()
    out = scaled_dot_product_attention(q1.cuda(), k.cuda(), v.cuda(), is_causal=True)
    exp = ref.sdpa(q1.double(), kr, vr, is_causal=True)
    assert_attn_close(out, exp, F32, "fp32 sdpa S_q != S_k")


def test_paged_layer_fp32_prefill_then_decode():
    """PagedCausalSelfAttention in fp32 (the reference's default dtype): prefill, then
    decode steps, against the reference pipeline restated in float64.  Module-level bar
    1e-4 (the PyTorch projections and norms around the kernels run in fp32 too)."""
    torch.manual_seed(5)
    hidden, heads, kv, hd, bs, nb = 512, 4, 2, 128, 16, 64
    m = PagedCausalSelfAttention(hidden, heads, num_kv_heads=kv, head_dim=hd, use_qk_norm=True,
                                 rope_base=1e6).to("cuda", F32)
    m.layer_idx = 0
    from tests.test_gpu_layers import CpuLayer
    cpu = CpuLayer(m)
    kc_g = torch.zeros((1, nb, kv, bs, hd), dtype=F32, device="cuda")
    vc_g = torch.zeros_like(kc_g)
    kc_c = torch.zeros((nb, kv, bs, hd), dtype=torch.float64)
    vc_c = torch.zeros_like(kc_c)
    prompts = [5, 33, 17]
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(3)).tolist()
    blocks, off = [], 0
    for L in prompts:
        n = (L + 8 + bs - 1) // bs
        blocks.append(perm[off:off + n])
        off += n

    def step(queries, x):
        md = meta.build(queries)
        mdg = AttentionMetadata(context_lens=md["context_lens"].cuda(),
                                kv_block_tables=md["kv_block_tables"].cuda(),
                                slot_mapping=md["slot_mapping"].cuda(), k_cache=kc_g,
                                v_cache=vc_g, is_prefill=md["is_prefill"])
        with torch.no_grad():
            out = m(x.cuda(), md["position_ids"].cuda(), md["attention_mask"].cuda(), mdg)
        exp = cpu.forward(x.double(), md["position_ids"], md["attention_mask"], md, kc_c, vc_c,
                          md["is_prefill"])
        return out, exp

    def close(out, exp, what):
        d = (out.double().cpu() - exp).abs()
        assert d.max().item() <= 1e-4, f"{what}: max-abs {d.max().item():.3g}"

    x = torch.randn(3, max(prompts), hidden) * 0.5
    q_pf = [meta.Query(L, 0, meta.PREFILL, blocks[i], bs) for i, L in enumerate(prompts)]
    out, exp = step(q_pf, x)
    for i, L in enumerate(prompts):
        close(out[i, :L], exp[i, :L], f"fp32 prefill seq {i}")
    for t in range(1, 3):
        xd = torch.randn(3, 1, hidden) * 0.5
        q_dec = [meta.Query(L, t, meta.DECODE, blocks[i], bs) for i, L in enumerate(prompts)]
        out, exp = step(q_dec, xd)
        close(out, exp, f"fp32 decode step {t}")
