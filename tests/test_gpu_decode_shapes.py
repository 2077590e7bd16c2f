"""Paged decode over the layouts the reference's configuration allows: block sizes other
than 16, powers of two or not (src/nano_inference/core/config.py:54 makes it a setting),
head dims 64 / 80 / 96,
any group (more than 16 query heads per KV head run as launches of at most 16 heads
each), KV head counts whose groups of the split kernel take 1, 2 or 4 heads per
workgroup, batches beyond the in-LDS unit prefix, and pools with invalid block ids.

Oracle: oracle.textbook (softmax(q K^T / sqrt(D)) V over keys [0, context_len) gathered
through the block table, head h -> KV head h // G), the mathematics of
src/nano_inference/layers/attention.py:285-332.  Bars: bf16 max-abs 2e-2 / mean-abs
2e-3; fp32 max-abs 1e-5.
"""
import math

import numpy as np
import pytest
import torch

from nano_inference_amd import ops, workloads
from oracle import textbook as tb
from tests.tolerances import assert_attn_close

pytestmark = pytest.mark.gpu


def oracle(c, seqs=None):
    b, h, d = c.q.shape
    hkv = c.num_kv_heads
    g = h // hkv
    bs = c.block_size
    q = c.q.double().cpu().numpy()
    seqs = range(b) if seqs is None else seqs
    out = np.zeros((len(seqs), h, d))
    for n, i in enumerate(seqs):
        L = c.lens[i]
        if L <= 0:
            continue
        ids = torch.tensor(c.tables_list[i], device=c.k_cache.device)
        kb = c.k_cache[0][ids].double().cpu().numpy()
        vb = c.v_cache[0][ids].double().cpu().numpy()
        kk = kb.transpose(1, 0, 2, 3).reshape(hkv, -1, d)[:, :L]
        vv = vb.transpose(1, 0, 2, 3).reshape(hkv, -1, d)[:, :L]
        for hk in range(hkv):
            out[n, hk * g:(hk + 1) * g] = tb.attend(q[i, hk * g:(hk + 1) * g], kk[hk], vv[hk],
                                                    1.0 / math.sqrt(d))
    return out


def step(c):
    ops.kv_write(c.k_new, c.v_new, c.k_cache[0], c.v_cache[0], c.slot_mapping)
    out = ops.paged_decode(c.q, c.k_cache[0], c.v_cache[0], c.block_tables, c.context_lens)
    torch.cuda.synchronize()
    return out


def edge_lens(bs):
    """Contexts on both sides of block and 32-key unit edges, plus long ones."""
    return [1, 2, bs - 1 if bs > 1 else 3, bs, bs + 1, 31, 32, 33, 2 * bs + 1, 600, 1333, 4100]


@pytest.mark.parametrize("bs", [4, 8, 32, 64, 128])
def test_bf16_block_sizes(bs):
    lens = edge_lens(bs)
    c = workloads.make_decode(len(lens), 16, 4, 128, lens, sum(-(-L // bs) for L in lens) + 9, bs,
                              torch.bfloat16, "cuda", seed=1200 + bs)
    assert_attn_close(step(c), oracle(c), torch.bfloat16, f"bf16 block size {bs}")


@pytest.mark.parametrize("bs,head_dim,hkv,group", [(12, 128, 4, 4), (24, 128, 2, 7),
                                                   (48, 80, 2, 2), (5, 64, 1, 3),
                                                   (2, 96, 2, 20), (1, 128, 8, 1),
                                                   (100, 128, 1, 16)])
def test_bf16_block_sizes_not_powers_of_two(bs, head_dim, hkv, group):
    """Block sizes that are not powers of two (the reference's is any positive integer):
    multiples of 4 (12, 24, 48, 100) on the split kernels, whose key-to-block step is a
    multiply-shift division, the rest (5, 2, 1) on the any-size kernel over the bf16 rows, at
    several head dims and groups (20 beyond the split kernels' 16 MFMA columns)."""
    lens = edge_lens(bs)
    c = workloads.make_decode(len(lens), hkv * group, hkv, head_dim, lens,
                              sum(-(-L // bs) for L in lens) + 9, bs, torch.bfloat16, "cuda",
                              seed=1290 + bs + head_dim)
    assert_attn_close(step(c), oracle(c), torch.bfloat16, f"bf16 bs={bs} D={head_dim} G={group}")


@pytest.mark.parametrize("head_dim", [64, 80, 96])
@pytest.mark.parametrize("bs", [8, 16])
def test_bf16_head_dims(head_dim, bs):
    lens = edge_lens(bs)
    c = workloads.make_decode(len(lens), 8, 2, head_dim, lens, sum(-(-L // bs) for L in lens) + 5,
                              bs, torch.bfloat16, "cuda", seed=1210 + head_dim + bs)
    assert_attn_close(step(c), oracle(c), torch.bfloat16, f"bf16 D={head_dim} bs={bs}")


@pytest.mark.parametrize("hkv,group", [(1, 16), (1, 5), (2, 12), (3, 4), (6, 2), (12, 1),
                                       (16, 2), (4, 16)])
def test_bf16_kv_head_counts_and_groups(hkv, group):
    """KV head counts whose workgroups take 4, 2 or 1 heads (1 .. 4 waves per head over
    separate key ranges) and groups up to 16 query heads."""
    lens = [5, 77, 1000, 2047, 33, 0, 300]
    c = workloads.make_decode(len(lens), hkv * group, hkv, 128, [max(L, 1) for L in lens], 512,
                              16, torch.bfloat16, "cuda", seed=1220 + 17 * hkv + group)
    ops.kv_write(c.k_new, c.v_new, c.k_cache[0], c.v_cache[0], c.slot_mapping)
    ctx = torch.tensor(lens, dtype=torch.int64, device="cuda")  # one empty context
    out = ops.paged_decode(c.q, c.k_cache[0], c.v_cache[0], c.block_tables, ctx)
    torch.cuda.synchronize()
    assert out[5].eq(0).all()
    c.lens = lens
    assert_attn_close(out, oracle(c), torch.bfloat16, f"H_kv={hkv} G={group}")


@pytest.mark.parametrize("hkv,group", [(1, 32), (2, 20), (1, 17), (4, 48)])
def test_bf16_groups_beyond_16(hkv, group):
    """More than 16 query heads per KV head (multi-query attention and wide GQA): the
    reference repeats each KV head G times (src/nano_inference/layers/attention.py:
    310-314), any G; here the heads run 16 at a time over the same keys.  One empty
    context and a batch of 1100 (unit prefix in the workspace) for one of them."""
    lens = [5, 77, 1000, 2047, 33, 0, 300]
    c = workloads.make_decode(len(lens), hkv * group, hkv, 128, [max(L, 1) for L in lens], 512,
                              16, torch.bfloat16, "cuda", seed=1240 + 17 * hkv + group)
    ops.kv_write(c.k_new, c.v_new, c.k_cache[0], c.v_cache[0], c.slot_mapping)
    ctx = torch.tensor(lens, dtype=torch.int64, device="cuda")
    out = ops.paged_decode(c.q, c.k_cache[0], c.v_cache[0], c.block_tables, ctx)
    torch.cuda.synchronize()
    assert out[5].eq(0).all()
    c.lens = lens
    assert_attn_close(out, oracle(c), torch.bfloat16, f"H_kv={hkv} G={group}")
    if group == 20:
        lens = [int(x) for x in torch.randint(1, 41, (1100,),
                                              generator=torch.Generator().manual_seed(5))]
        c = workloads.make_decode(1100, hkv * group, hkv, 128, lens, 4096, 16, torch.bfloat16,
                                  "cuda", seed=1250, max_blocks=4)
        assert_attn_close(step(c), oracle(c), torch.bfloat16, f"G={group} batch 1100")


@pytest.mark.parametrize("batch", [1, 3])
def test_bf16_one_long_sequence_over_many_ranges(batch):
    """A 64k-token context cut over every wave of the grid (combine of hundreds of
    partials), alone and beside two short ones."""
    lens = [65536, 17, 1][:batch]
    c = workloads.make_decode(batch, 8, 8, 128, lens, 4200, 16, torch.bfloat16, "cuda", seed=1230)
    assert_attn_close(step(c), oracle(c), torch.bfloat16, f"64k context, batch {batch}")


@pytest.mark.parametrize("hkv,lens", [(8, [1000, 37]), (1, [3000, 1, 5]), (2, [64, 33, 1, 500])])
def test_bf16_fewer_units_than_ranges(hkv, lens):
    """Fewer 32-key units than the grid has ranges: most ranges are empty, and a sequence's
    units lie in ranges with empty ones between them, whose slots the merge reads as "no
    keys"; the merge takes the first and last range from the split kernel's records."""
    c = workloads.make_decode(len(lens), 2 * hkv, hkv, 128, lens, 400, 16, torch.bfloat16,
                              "cuda", seed=1235 + hkv)
    assert_attn_close(step(c), oracle(c), torch.bfloat16, f"few units, H_kv {hkv}")


def test_bf16_batch_beyond_the_lds_prefix():
    """3000 sequences: the unit prefix is built by its own kernel; many sequences per
    range (checked on a sample of 60)."""
    g = torch.Generator().manual_seed(1240)
    lens = [int(x) for x in torch.randint(1, 200, (3000,), generator=g)]
    c = workloads.make_decode(3000, 8, 2, 128, lens, sum(-(-L // 16) for L in lens) + 3, 16,
                              torch.bfloat16, "cuda", seed=1240, max_blocks=16)
    out = step(c)
    seqs = list(range(0, 3000, 50))
    assert_attn_close(out[seqs], oracle(c, seqs), torch.bfloat16, "batch 3000")


def test_bf16_invalid_block_ids_are_skipped():
    """Table entries outside [0, num_blocks) contribute nothing (neither their scores nor
    their values), at block sizes 8 and 32."""
    for bs in (8, 32):
        lens = [200, 64, 129]
        c = workloads.make_decode(3, 8, 2, 128, lens, 64, bs, torch.bfloat16, "cuda",
                                  seed=1250 + bs)
        ops.kv_write(c.k_new, c.v_new, c.k_cache[0], c.v_cache[0], c.slot_mapping)
        bt = c.block_tables.clone()
        bad = {0: [1], 2: [0, 3]}
        for s, cols in bad.items():
            for col in cols:
                bt[s, col] = -5 if col % 2 else 10 ** 6
        out = ops.paged_decode(c.q, c.k_cache[0], c.v_cache[0], bt, c.context_lens)
        torch.cuda.synchronize()
        # oracle: the same keys without the skipped blocks' rows
        q = c.q.double().cpu().numpy()
        exp = np.zeros_like(q)
        for s, L in enumerate(lens):
            keep = [t for t in range(L) if t // bs not in bad.get(s, [])]
            ids = np.asarray(c.tables_list[s])
            t = np.asarray(keep)
            kc = c.k_cache[0].double().cpu().numpy()[ids[t // bs], :, t % bs]  # (n, H_kv, D)
            vc = c.v_cache[0].double().cpu().numpy()[ids[t // bs], :, t % bs]
            for hk in range(2):
                exp[s, 4 * hk:4 * hk + 4] = tb.attend(q[s, 4 * hk:4 * hk + 4], kc[:, hk],
                                                      vc[:, hk], 1 / math.sqrt(128))
        assert_attn_close(out, exp, torch.bfloat16, f"invalid ids bs={bs}")


@pytest.mark.parametrize("bs", [32, 64, 48, 8, 12, 24, 1])
def test_fp8_block_sizes(bs):
    """fp8 caches at block sizes 32, 64 and 48 (split kernels: multiples of 16, a tile in
    one block) and 8, 12, 24, 1 (the any-size kernel, rows dequantised on load)."""
    from tests.test_gpu_fp8_kv import oracle_decode_fp8
    lens = edge_lens(bs)
    c = workloads.make_decode(len(lens), 16, 4, 128, lens, sum(-(-L // bs) for L in lens) + 9, bs,
                              torch.bfloat16, "cuda", seed=1260 + bs)
    ops.kv_write(c.k_new, c.v_new, c.k_cache[0], c.v_cache[0], c.slot_mapping)
    f8 = workloads.quantize_cache_fp8(c)
    out = ops.paged_decode(c.q, f8.k_cache[0], f8.v_cache[0], c.block_tables, c.context_lens,
                           k_scale=f8.k_scale[0], v_scale=f8.v_scale[0])
    torch.cuda.synchronize()
    assert_attn_close(out, oracle_decode_fp8(c, f8), torch.bfloat16, f"fp8 block size {bs}")


@pytest.mark.parametrize("head_dim,bs,hkv,group", [(128, 8, 4, 2), (128, 32, 2, 4),
                                                   (64, 16, 2, 4), (80, 16, 4, 1),
                                                   (96, 5, 2, 2), (128, 16, 1, 12)])
def test_fp32_other_layouts(head_dim, bs, hkv, group):
    """fp32 decode outside head_dim 128 / block 16 / groups <= 8 (the fp32 prefill kernel
    with one query row per sequence)."""
    lens = edge_lens(bs)
    c = workloads.make_decode(len(lens), hkv * group, hkv, head_dim, lens,
                              sum(-(-L // bs) for L in lens) + 4, bs, torch.float32, "cuda",
                              seed=1270 + head_dim + bs)
    assert_attn_close(step(c), oracle(c), torch.float32, f"fp32 D={head_dim} bs={bs} G={group}")


def test_unsupported_layouts_raise_before_launch():
    c = workloads.make_decode(2, 8, 2, 112, [5, 9], 8, 16, torch.bfloat16, "cuda", seed=1280)
    with pytest.raises(ValueError, match="head_dim"):
        ops.paged_decode(c.q, c.k_cache[0], c.v_cache[0], c.block_tables, c.context_lens)
    ops.check_decode_shape(128, 16, 32, 1)  # any group
    ops.check_decode_shape(128, 2, 32, 1)  # any block size
    ops.check_decode_shape(128, 2, 32, 1, torch.float32)
