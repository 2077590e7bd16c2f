"""Seeded random shapes for the decode, prefill and chunked-prefill kernels vs the float64
oracle, every output row checked.

Each seed draws one configuration from the layouts the kernels take: batch and sequence
counts, KV-head counts and query heads per KV head (GQA groups 1..16), head_dim 64 / 80 /
96 / 128, KV block sizes 4..256, context and query lengths with block-, unit- and
tile-edge values forced in (1, 15, 16, 17, 31, 32, 33, 63, 64, 65, block size +- 1), and
for prefill the three masks (top-left causal, bottom-right causal after earlier keys, none,
including empty sequences).  The configuration is printed before the call, so a failure
names it.  Oracles: oracle.textbook.paged_decode / varlen / attend (softmax(q K^T * scale)
V with an explicit visible-key bound per row), fp8 caches dequantised by oracle.fp8_kv.
Bars: bf16 max-abs 2e-2, mean-abs 2e-3 (tests/tolerances.py).
"""
import math
import random

import numpy as np
import pytest
import torch

from nano_inference_amd import ops, workloads
from oracle import fp8_kv as F
from oracle import textbook as tb
from tests.test_gpu_prefill import _chunk_oracle
from tests.tolerances import assert_attn_close

pytestmark = pytest.mark.gpu

EDGE_LENS = [1, 15, 16, 17, 31, 32, 33, 63, 64, 65]


def _lengths(rng, n, lo, hi, extra=()):
    pool = [x for x in list(EDGE_LENS) + list(extra) if lo <= x <= hi]
    return [rng.choice(pool) if pool and rng.random() < 0.4 else rng.randint(lo, hi)
            for _ in range(n)]


@pytest.mark.parametrize("seed", range(16))
def test_random_decode(seed):
    rng = random.Random(1000 + seed)
    fp8 = seed % 4 == 3
    d = 128 if fp8 else rng.choice([64, 80, 96, 128])
    bs = rng.choice([16, 32, 64, 128] if fp8 else [4, 8, 16, 32, 64, 128, 256])
    hkv = rng.choice([1, 2, 4, 8])
    group = rng.choice([1, 2, 3, 4, 5, 7, 8, 12, 16])
    batch = rng.randint(1, 32)
    lens = _lengths(rng, batch, 1, 2000, extra=(bs - 1, bs, bs + 1, 2 * bs))
    pool = sum(math.ceil(L / bs) for L in lens) + 8
    print(f"decode seed {seed}: fp8 {fp8} D {d} bs {bs} hkv {hkv} G {group} batch {batch} "
          f"lens {lens}", flush=True)
    c = workloads.make_decode(batch, hkv * group, hkv, d, lens, pool, bs, torch.bfloat16,
                              "cuda", seed=2000 + seed)
    scale = 1.0 / math.sqrt(d)
    bt, cl = c.block_tables.cpu().numpy(), c.context_lens.cpu().numpy()
    q = c.q.double().cpu().numpy()
    if fp8:
        f8 = workloads.quantize_cache_fp8(c)
        out = ops.paged_decode(c.q, f8.k_cache[0], f8.v_cache[0], c.block_tables,
                               c.context_lens, k_scale=f8.k_scale[0], v_scale=f8.v_scale[0])
        kd = F.dequantize_rows(f8.k_cache[0].cpu(), f8.k_scale[0].cpu()).double().numpy()
        vd = F.dequantize_rows(f8.v_cache[0].cpu(), f8.v_scale[0].cpu()).double().numpy()
    else:
        out = ops.paged_decode(c.q, c.k_cache[0], c.v_cache[0], c.block_tables,
                               c.context_lens)
        kd = c.k_cache[0].double().cpu().numpy()
        vd = c.v_cache[0].double().cpu().numpy()
    torch.cuda.synchronize()
    exp = tb.paged_decode(q, kd, vd, bt, cl, scale)
    assert_attn_close(out, exp, torch.bfloat16, f"decode seed {seed}")


@pytest.mark.parametrize("seed", range(16))
def test_random_prefill(seed):
    rng = random.Random(3000 + seed)
    d = rng.choice([64, 80, 96, 128])
    hkv = rng.choice([1, 2, 4])
    group = rng.choice([1, 2, 4, 7])
    mode = rng.choice(["top_left", "none", "bottom_right"])
    n = rng.randint(1, 10)
    ql = _lengths(rng, n, 0 if mode == "none" else 1, 400, extra=(127, 128, 129))
    if mode == "bottom_right":
        kl = [q + rng.choice([0, 1, 16, 64, rng.randint(0, 500)]) for q in ql]
    else:
        kl = list(ql)
    print(f"prefill seed {seed}: mode {mode} D {d} hkv {hkv} G {group} q {ql} k {kl}",
          flush=True)
    g = torch.Generator().manual_seed(4000 + seed)
    h = hkv * group
    tq, tk = max(sum(ql), 1), max(sum(kl), 1)
    q = torch.randn(tq, h, d, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(tk, hkv, d, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(tk, hkv, d, generator=g).to(torch.bfloat16).cuda()
    qs = torch.tensor([0] + ql[:-1]).cumsum(0).to(torch.int32).cuda()
    ks = torch.tensor([0] + kl[:-1]).cumsum(0).to(torch.int32).cuda()
    qlt = torch.tensor(ql, dtype=torch.int32).cuda()
    klt = torch.tensor(kl, dtype=torch.int32).cuda()
    code = {"top_left": ops.CAUSAL_TOP_LEFT, "none": ops.CAUSAL_NONE,
            "bottom_right": ops.CAUSAL_BOTTOM_RIGHT}[mode]
    out = ops.prefill(q, k, v, qs, qlt, ks, klt, max(max(ql), 1), code)
    torch.cuda.synchronize()
    res = tb.varlen(q.double().cpu().numpy(), k.double().cpu().numpy(),
                    v.double().cpu().numpy(), qs.cpu().numpy(), ql, ks.cpu().numpy(), kl,
                    1.0 / math.sqrt(d), mode)
    o = out.double().cpu().numpy()
    got = [o[int(qs[s]) + idx] for s, (idx, _) in res.items() if len(idx)]
    exp = [ref for _, (idx, ref) in res.items() if len(idx)]
    if got:
        assert_attn_close(np.concatenate(got), np.concatenate(exp), torch.bfloat16,
                          f"prefill seed {seed}")


@pytest.mark.parametrize("seed", range(10))
def test_random_chunked_prefill(seed):
    rng = random.Random(5000 + seed)
    bs = rng.choice([4, 8, 16, 32, 64, 128, 256])
    hkv = rng.choice([1, 2, 4])
    group = rng.choice([1, 2, 4, 8])
    n = rng.randint(1, 6)
    chunk = rng.choice([1, 17, 64, 65, 128, 200])
    prior = [rng.choice([0, 1, bs - 1, bs, bs + 1, rng.randint(0, 1500)]) for _ in range(n)]
    print(f"chunked seed {seed}: bs {bs} hkv {hkv} G {group} chunk {chunk} prior {prior}",
          flush=True)
    c = workloads.chunked_qwen3_8b("cuda", seed=6000 + seed, n=n, chunk=chunk, prior=prior,
                                   num_heads=hkv * group, num_kv_heads=hkv, block_size=bs)
    out = ops.prefill_paged(c.q, c.k_cache, c.v_cache, c.block_tables, c.q_start, c.q_len,
                            c.context_lens, c.chunk)
    torch.cuda.synchronize()
    o = out.double().cpu().numpy()
    for s, (idx, ref) in _chunk_oracle(c, None).items():
        assert_attn_close(o[s * c.chunk + idx], ref, torch.bfloat16, f"chunked seed {seed} seq {s}")
