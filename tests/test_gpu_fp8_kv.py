"""fp8 KV cache (e4m3 codes + one fp32 scale per row) on the GPU vs the oracle.

- KV write (nia_kv_write_fp8) and the fused QK kernel's fp8 write: codes and scales
  bit for bit equal to oracle.fp8_kv (the reference's write loop,
  src/nano_inference/layers/attention.py:267-278, with each row quantised).
- Paged decode over fp8 caches (nia_paged_decode_fp8) vs the float64 textbook
  attention over the dequantised caches (code * scale): the bf16 bar, max-abs
  <= 2e-2 and mean-abs <= 2e-3.  Garbage past the context (NaN codes, NaN scales)
  must not leak; a zero-length context gives zeros.
"""
import math

import numpy as np
import pytest
import torch

from nano_inference_amd import ops, workloads
from oracle import fp8_kv as F
from oracle import metadata as meta
from oracle import qk_rope as O
from oracle import textbook as tb
from tests.tolerances import assert_attn_close

pytestmark = pytest.mark.gpu


def fp8_pool(nb, hkv, bs=16, d=128, device="cuda"):
    return (torch.zeros((nb, hkv, bs, d), dtype=torch.uint8, device=device),
            torch.zeros((nb, hkv, bs, d), dtype=torch.uint8, device=device),
            torch.zeros((nb, hkv, bs), dtype=torch.float32, device=device),
            torch.zeros((nb, hkv, bs), dtype=torch.float32, device=device))


def check_write(k, v, slots, nb, bs=16):
    hkv = k.shape[-2]
    kc, vc, ks, vs = fp8_pool(nb, hkv, bs)
    ops.kv_write(k, v, kc, vc, slots, ks, vs)
    torch.cuda.synchronize()
    ekc, evc, eks, evs = (t.cpu() for t in fp8_pool(nb, hkv, bs, device="cpu"))
    F.kv_write_loop_fp8(k.cpu().reshape(slots.shape + k.shape[-2:]),
                        v.cpu().reshape(slots.shape + v.shape[-2:]), ekc, evc, eks, evs,
                        slots.cpu())
    assert torch.equal(kc.cpu(), ekc) and torch.equal(vc.cpu(), evc), "codes"
    assert torch.equal(ks.cpu().view(torch.int32), eks.view(torch.int32)), "k scales"
    assert torch.equal(vs.cpu().view(torch.int32), evs.view(torch.int32)), "v scales"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_write_decode_step(dtype):
    g = torch.Generator(device="cuda").manual_seed(1)
    k = (torch.randn((64, 1, 8, 128), generator=g, device="cuda") * 3).to(dtype)
    v = torch.randn((64, 1, 8, 128), generator=g, device="cuda").to(dtype)
    k[3, 0, 2] = 0  # a zero row: scale 0, zero codes
    slots = torch.randperm(512 * 16, generator=torch.Generator().manual_seed(2))[:64]
    check_write(k, v, slots.view(64, 1).cuda(), 512)


def test_write_padded_prefill_with_negative_and_out_of_range_slots():
    lens = [37, 5, 64]
    bs, nb = 16, 32
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(3)).tolist()
    qs, off = [], 0
    for L in lens:
        n = -(-L // bs)
        qs.append(meta.Query(L, 0, meta.PREFILL, perm[off:off + n], bs))
        off += n
    md = meta.build(qs)
    slots = md["slot_mapping"].clone()
    slots[2, 63] = nb * bs + 5  # past the pool: skipped
    g = torch.Generator(device="cuda").manual_seed(4)
    b, s = slots.shape
    k = torch.randn((b, s, 4, 128), generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn((b, s, 4, 128), generator=g, device="cuda").to(torch.bfloat16)
    kc, vc, ks, vs = fp8_pool(nb, 4, bs)
    ops.kv_write(k, v, kc, vc, slots.cuda(), ks, vs)
    torch.cuda.synchronize()
    ekc, evc, eks, evs = fp8_pool(nb, 4, bs, device="cpu")
    ok = slots.clone()
    ok[ok >= nb * bs] = -1
    F.kv_write_loop_fp8(k.cpu(), v.cpu(), ekc, evc, eks, evs, ok)
    assert torch.equal(kc.cpu(), ekc) and torch.equal(vc.cpu(), evc)
    assert torch.equal(ks.cpu(), eks) and torch.equal(vs.cpu(), evs)


def test_fused_qk_write_fp8():
    g = torch.Generator().manual_seed(5)
    n, h, hkv, nb = 40, 16, 8, 8
    q = torch.randn(n, h, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(n, hkv, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(n, hkv, 128, generator=g).to(torch.bfloat16)
    qw = (torch.randn(128, generator=g) * 0.3 + 1).to(torch.bfloat16)
    kw = (torch.randn(128, generator=g) * 0.3 + 1).to(torch.bfloat16)
    pos = torch.randint(0, 5000, (n,), generator=g)
    slots = torch.randperm(nb * 16, generator=g)[:n]
    slots[7] = -1
    kc, vc, ks, vs = fp8_pool(nb, hkv)
    qg, kg, vg = q.cuda(), k.cuda(), v.cuda()
    ops.qk_norm_rope_kv_write(qg, kg, vg, qw.cuda(), kw.cuda(), 1e-6, pos.cuda(),
                              O.inv_freq(128, 1e6).cuda(), None, kc, vc, slots.cuda(), ks, vs)
    torch.cuda.synchronize()
    ekc, evc, eks, evs = fp8_pool(nb, hkv, device="cpu")
    F.kv_write_loop_fp8(kg.cpu().view(1, n, hkv, 128), v.view(1, n, hkv, 128), ekc, evc, eks,
                        evs, slots.view(1, n))
    assert torch.equal(kc.cpu(), ekc) and torch.equal(vc.cpu(), evc)
    assert torch.equal(ks.cpu(), eks) and torch.equal(vs.cpu(), evs)


def oracle_decode_fp8(c, f8, layer=0, seqs=None):
    b, h, d = c.q.shape
    hkv = c.num_kv_heads
    gq = h // hkv
    q = c.q.double().cpu().numpy()
    out = np.zeros((b, h, d))
    scale = 1.0 / math.sqrt(d)
    for i in range(b) if seqs is None else seqs:
        L = c.lens[i]
        if L == 0:
            continue
        ids = torch.tensor(c.tables_list[i], device="cuda")
        kb = F.dequantize_rows(f8.k_cache[layer][ids].cpu(), f8.k_scale[layer][ids].cpu())
        vb = F.dequantize_rows(f8.v_cache[layer][ids].cpu(), f8.v_scale[layer][ids].cpu())
        kk = kb.double().numpy().transpose(1, 0, 2, 3).reshape(hkv, -1, d)[:, :L]
        vv = vb.double().numpy().transpose(1, 0, 2, 3).reshape(hkv, -1, d)[:, :L]
        for hk in range(hkv):
            out[i, hk * gq:(hk + 1) * gq] = tb.attend(q[i, hk * gq:(hk + 1) * gq], kk[hk],
                                                      vv[hk], scale)
    return out


def run_fp8(c, f8, layer=0):
    out = ops.paged_decode(c.q, f8.k_cache[layer], f8.v_cache[layer], c.block_tables,
                           c.context_lens, k_scale=f8.k_scale[layer], v_scale=f8.v_scale[layer])
    torch.cuda.synchronize()
    return out


def test_decode_fp8_small():
    c = workloads.decode_small("cuda", torch.bfloat16)
    f8 = workloads.quantize_cache_fp8(c)
    assert_attn_close(run_fp8(c, f8), oracle_decode_fp8(c, f8), torch.bfloat16, "fp8 small")


@pytest.mark.parametrize("g", [1, 2, 4, 7, 8, 16, 24, 32])
def test_decode_fp8_group_sizes(g):
    lens = [1, 15, 16, 17, 300, 513, 1100]
    c = workloads.make_decode(len(lens), 2 * g, 2, 128, lens, 256, 16, torch.bfloat16, "cuda",
                              seed=70 + g)
    f8 = workloads.quantize_cache_fp8(c)
    assert_attn_close(run_fp8(c, f8), oracle_decode_fp8(c, f8), torch.bfloat16, f"fp8 G={g}")


@pytest.mark.parametrize("batch", [1024, 1025])
@pytest.mark.parametrize("heads", [16, 28])
def test_decode_fp8_at_the_staged_batch_limit(heads, batch):
    """fp8 batches of up to 1024 sequences build the split kernel's unit prefix in LDS;
    above it decode_prefix_kernel writes it to the workspace first.  Groups of 4 and 7,
    short contexts (1 to 40 tokens) keep the oracle quick."""
    lens = [int(x) for x in torch.randint(1, 41, (batch,),
                                          generator=torch.Generator().manual_seed(batch + 7))]
    c = workloads.make_decode(batch, heads, 4, 128, lens, 4096, 16, torch.bfloat16, "cuda",
                              seed=batch + 7, max_blocks=4)
    f8 = workloads.quantize_cache_fp8(c)
    assert_attn_close(run_fp8(c, f8), oracle_decode_fp8(c, f8), torch.bfloat16,
                      f"fp8 G={heads // 4} batch {batch}")


def test_decode_fp8_rejects_scales_off_a_16_byte_boundary():
    """The decode reads a block-head's row scales 16 bytes at a time: a scale tensor that
    starts 4 bytes into an allocation is refused before any launch."""
    c = workloads.make_decode(2, 8, 2, 128, [40, 70], 16, 16, torch.bfloat16, "cuda", seed=3)
    f8 = workloads.quantize_cache_fp8(c)
    ks = f8.k_scale[0]
    shifted = torch.empty(ks.numel() + 1, dtype=torch.float32, device="cuda")[1:].view(ks.shape)
    shifted.copy_(ks)
    with pytest.raises(RuntimeError, match="(?i)align"):
        ops.paged_decode(c.q, f8.k_cache[0], f8.v_cache[0], c.block_tables, c.context_lens,
                         k_scale=shifted, v_scale=f8.v_scale[0])
    torch.cuda.synchronize()


def test_decode_fp8_qwen3_8b_sampled_rows():
    """The 64-sequence Qwen3-8B workload; every row checked on 12 sequences."""
    c = workloads.decode_qwen3_8b("cuda")
    f8 = workloads.quantize_cache_fp8(c)
    out = run_fp8(c, f8)
    seqs = list(range(0, 64, 6))
    exp = oracle_decode_fp8(c, f8, seqs=seqs)
    assert_attn_close(out[seqs], exp[seqs], torch.bfloat16, "fp8 qwen3-8b")


def test_decode_fp8_ignores_garbage_past_the_context_and_empty_contexts():
    lens = [5, 9, 40, 161]
    c = workloads.make_decode(len(lens), 8, 2, 128, lens, 64, 16, torch.bfloat16, "cuda",
                              seed=91, max_blocks=12)
    f8 = workloads.quantize_cache_fp8(c)
    ctx = c.context_lens.clone()
    ctx[0] = 0
    live = [0] + lens[1:]
    # poison every slot past each context in the sequences' own blocks
    for i, L in enumerate(live):
        for j, blk in enumerate(c.tables_list[i]):
            for t in range(16):
                if j * 16 + t >= L:
                    f8.k_cache[0, blk, :, t] = 0x7F
                    f8.v_cache[0, blk, :, t] = 0x7F
                    f8.k_scale[0, blk, :, t] = float("nan")
                    f8.v_scale[0, blk, :, t] = float("nan")
    out = ops.paged_decode(c.q, f8.k_cache[0], f8.v_cache[0], c.block_tables, ctx,
                           k_scale=f8.k_scale[0], v_scale=f8.v_scale[0])
    torch.cuda.synchronize()
    assert torch.all(out[0] == 0)
    exp = oracle_decode_fp8(c, f8, seqs=[1, 2, 3])
    assert_attn_close(out[1:], exp[1:], torch.bfloat16, "fp8 poisoned")


def test_chunked_prefill_over_fp8_cache():
    """Chunks on top of an fp8 cache (dequantising gather + varlen prefill) vs the float64
    textbook over the dequantised cache, on a fixed sample of query rows per chunk."""
    c = workloads.chunked_qwen3_8b("cuda", n=3)
    nb, hkv, bs, d = c.k_cache.shape
    kc, vc, ks, vs = fp8_pool(nb, hkv, bs)
    slots = torch.arange(nb * bs, dtype=torch.int64, device="cuda")
    ops.kv_write(c.k_cache.transpose(1, 2).reshape(nb * bs, hkv, d),
                 c.v_cache.transpose(1, 2).reshape(nb * bs, hkv, d), kc, vc, slots, ks, vs)
    out = ops.prefill_paged(c.q, kc, vc, c.block_tables, c.q_start, c.q_len, c.context_lens,
                            c.chunk, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    kd = F.dequantize_rows(kc.cpu(), ks.cpu()).double().numpy()
    vd = F.dequantize_rows(vc.cpu(), vs.cpu()).double().numpy()
    res = tb.paged_prefill(c.q.double().cpu().numpy(), kd, vd, c.block_tables.cpu().numpy(),
                           c.q_start.cpu().numpy(), c.q_len.cpu().numpy(),
                           c.context_lens.cpu().numpy(), 1.0 / math.sqrt(d),
                           rows={i: [0, 1, 63, 64, 127, 128, 255, 300, 447, 510, 511]
                                 for i in range(3)})
    got = out.cpu()
    for s_, (idx, o) in res.items():
        rows = got[int(c.q_start[s_]) + torch.as_tensor(idx)]
        assert_attn_close(rows, o, torch.bfloat16, f"chunk {s_} over fp8")


def test_paged_layer_with_fp8_cache_matches_reference_pipeline():
    """PagedCausalSelfAttention over fp8 caches: prefill (attends to the fresh K/V, writes
    the cache) then decode steps (read the cache) vs the reference pipeline in float64
    whose cache holds the dequantised rows."""
    from nano_inference_amd import AttentionMetadata, PagedCausalSelfAttention
    from oracle import reference_attention as ref
    from tests.test_gpu_layers import CpuLayer, close

    torch.manual_seed(0)
    hidden, heads, kv, hd, bs, nb = 512, 4, 2, 128, 16, 64
    m = PagedCausalSelfAttention(hidden, heads, num_kv_heads=kv, head_dim=hd, use_qk_norm=True,
                                 rope_base=1e6).to("cuda", torch.bfloat16)
    m.layer_idx = 0
    cpu = CpuLayer(m)
    kc = torch.zeros((1, nb, kv, bs, hd), dtype=torch.uint8, device="cuda")
    vc = torch.zeros_like(kc)
    ks = torch.zeros((1, nb, kv, bs), dtype=torch.float32, device="cuda")
    vs = torch.zeros_like(ks)
    kc_c = torch.zeros((nb, kv, bs, hd), dtype=torch.float64)
    vc_c = torch.zeros_like(kc_c)
    prompts = [5, 33, 17]
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(3)).tolist()
    blocks, off = [], 0
    for L in prompts:
        n = (L + 8 + bs - 1) // bs
        blocks.append(perm[off:off + n])
        off += n

    def qdq(t):  # quantise-dequantise rows as the fp8 cache stores them
        codes, sc = F.quantize_rows(t.to(torch.bfloat16))
        return F.dequantize_rows(codes, sc).double()

    def cpu_step(x, md, prefill):
        sd = cpu.sd
        b, s_, _ = x.shape
        q = (x @ sd["q_proj.weight"].T).view(b, s_, heads, hd)
        k = (x @ sd["k_proj.weight"].T).view(b, s_, kv, hd)
        v = (x @ sd["v_proj.weight"].T).view(b, s_, kv, hd)
        q, k = cpu.q_norm(q), cpu.k_norm(k)
        q, k = cpu.rot(q, k, md["position_ids"])
        if prefill:  # attention over the fresh rows, then the cache keeps their fp8 form
            attn = ref.paged_attention(q, k, v, kc_c, vc_c, md["slot_mapping"],
                                       md["kv_block_tables"], md["context_lens"],
                                       md["attention_mask"], True)
            ref.kv_write_loop(qdq(k), qdq(v), kc_c, vc_c, md["slot_mapping"])
        else:
            attn = ref.paged_attention(q, qdq(k), qdq(v), kc_c, vc_c, md["slot_mapping"],
                                       md["kv_block_tables"], md["context_lens"],
                                       md["attention_mask"], False)
        return attn.reshape(b, s_, -1) @ sd["o_proj.weight"].T

    def step(queries, x, prefill):
        md = meta.build(queries)
        mdg = AttentionMetadata(context_lens=md["context_lens"].cuda(),
                                kv_block_tables=md["kv_block_tables"].cuda(),
                                slot_mapping=md["slot_mapping"].cuda(), k_cache=kc, v_cache=vc,
                                is_prefill=md["is_prefill"], k_scale=ks, v_scale=vs)
        out = m(x.cuda(), md["position_ids"].cuda(), md["attention_mask"].cuda(), mdg)
        return out, cpu_step(x.double(), md, prefill)

    x = (torch.randn(3, max(prompts), hidden) * 0.5).to(torch.bfloat16)
    out, exp = step([meta.Query(L, 0, meta.PREFILL, blocks[i], bs)
                     for i, L in enumerate(prompts)], x, True)
    for i, L in enumerate(prompts):
        close(out[i, :L], exp[i, :L], f"prefill seq {i}")
    for t in range(1, 4):
        xd = (torch.randn(3, 1, hidden) * 0.5).to(torch.bfloat16)
        out, exp = step([meta.Query(L, t, meta.DECODE, blocks[i], bs)
                         for i, L in enumerate(prompts)], xd, False)
        close(out, exp, f"fp8 decode step {t}")
