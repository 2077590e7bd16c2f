"""Paged decode kernel vs the float64 oracle, plus closed forms and invariants.

Oracle: oracle.textbook (softmax(q K^T / sqrt(D)) V per sequence over keys
[0, context_len), head h -> KV head h // G), the mathematics of
src/nano_inference/layers/attention.py:285-332 and :12-50.
Bars: bf16 max-abs 2e-2 / mean-abs 2e-3, fp32 max-abs 1e-5.
"""
import math

import numpy as np
import pytest
import torch

from nano_inference_amd import ops, workloads
from oracle import textbook as tb
from tests.tolerances import assert_attn_close

pytestmark = pytest.mark.gpu


def oracle_decode(c: workloads.DecodeCase, layer: int = 0, seqs=None,
                  scale=None) -> np.ndarray:
    """Float64 oracle, streaming one sequence's blocks at a time from the GPU."""
    b, h, d = c.q.shape
    hkv = c.num_kv_heads
    g = h // hkv
    q = c.q.double().cpu().numpy()
    out = np.zeros((b, h, d))
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    for i in range(b) if seqs is None else seqs:
        L = c.lens[i]
        ids = torch.tensor(c.tables_list[i], device=c.k_cache.device)
        kb = c.k_cache[layer][ids].double().cpu().numpy()  # (n, H_kv, BS, D)
        vb = c.v_cache[layer][ids].double().cpu().numpy()
        kk = kb.transpose(1, 0, 2, 3).reshape(hkv, -1, d)[:, :L]
        vv = vb.transpose(1, 0, 2, 3).reshape(hkv, -1, d)[:, :L]
        for hk in range(hkv):
            out[i, hk * g:(hk + 1) * g] = tb.attend(q[i, hk * g:(hk + 1) * g], kk[hk], vv[hk], scale)
    return out


def run_step(c: workloads.DecodeCase, layer: int = 0) -> torch.Tensor:
    ops.kv_write(c.k_new, c.v_new, c.k_cache[layer], c.v_cache[layer], c.slot_mapping)
    out = ops.paged_decode(c.q, c.k_cache[layer], c.v_cache[layer], c.block_tables,
                           c.context_lens)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_small(dtype):
    """4 sequences, 16/8 heads, contexts 17/64/200/511, 128-block pool."""
    c = workloads.decode_small("cuda", dtype)
    out = run_step(c)
    assert_attn_close(out, oracle_decode(c), dtype, f"decode_small {dtype}")


def test_decode_qwen3_8b_full_batch():
    """64 sequences, 32/8 heads, contexts U[512, 8192], 40k-block shuffled pool."""
    c = workloads.decode_qwen3_8b("cuda")
    out = run_step(c)
    assert_attn_close(out, oracle_decode(c), torch.bfloat16, "decode_qwen3_8b")


def test_decode_vl_group_of_seven():
    """32 sequences, 28/4 heads (7 query heads per KV head), contexts U[1024, 6144]."""
    c = workloads.decode_vl("cuda")
    out = run_step(c)
    assert_attn_close(out, oracle_decode(c), torch.bfloat16, "decode_vl")


@pytest.mark.parametrize("group", [1, 2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_block_boundaries(group, dtype):
    lens = [1, 2, 15, 16, 17, 31, 32, 33, 511, 512, 513, 1025]
    hkv = 2
    c = workloads.make_decode(len(lens), hkv * group, hkv, 128, lens, 512, 16, dtype, "cuda",
                              seed=40 + group)
    out = run_step(c)
    assert_attn_close(out, oracle_decode(c), dtype, f"boundaries G={group}")


def test_long_contexts_and_a_zeroed_context():
    """A Qwen3-8B-wide batch (40 sequences x 8 KV heads, 512-block tables): contexts on
    both sides of 768-token multiples, a single token, a full table; then one context
    cut to zero after the write (its output is zeros; the others still match the oracle,
    though not bit for bit: the key ranges of the waves move with the total)."""
    lens = [1, 16, 17, 767, 768, 769, 1535, 1536, 1537, 2303, 2304, 2305, 8192, 8191, 4000]
    lens += [int(x) for x in torch.randint(1, 8193, (40 - len(lens),),
                                           generator=torch.Generator().manual_seed(48))]
    c = workloads.make_decode(len(lens), 32, 8, 128, lens, 40000, 16, torch.bfloat16, "cuda",
                              seed=480, max_blocks=512)
    out = run_step(c)
    exp = oracle_decode(c)
    assert_attn_close(out, exp, torch.bfloat16, "long contexts")
    ctx = c.context_lens.clone()
    ctx[5] = 0
    out0 = ops.paged_decode(c.q, c.k_cache[0], c.v_cache[0], c.block_tables, ctx)
    torch.cuda.synchronize()
    assert out0[5].eq(0).all()
    keep = [i for i in range(len(lens)) if i != 5]
    assert_attn_close(out0[keep], exp[keep], torch.bfloat16, "long contexts, one zeroed")


@pytest.mark.parametrize("batch", [1024, 1025])
@pytest.mark.parametrize("heads", [16, 28])
def test_groups_at_the_lds_prefix_batch_limit(heads, batch):
    """bf16 batches of up to 1024 sequences build the split kernel's unit prefix in LDS
    inside the kernel; above it decode_prefix_kernel writes the prefix to the workspace
    first and the split kernel reads it from there.  Groups of 4 and 7, short contexts
    (1 to 40 tokens) keep the oracle quick."""
    lens = [int(x) for x in torch.randint(1, 41, (batch,),
                                          generator=torch.Generator().manual_seed(batch))]
    c = workloads.make_decode(batch, heads, 4, 128, lens, 4096, 16, torch.bfloat16, "cuda",
                              seed=batch, max_blocks=4)
    out = run_step(c)
    assert_attn_close(out, oracle_decode(c), torch.bfloat16, f"G={heads // 4} batch {batch}")


def test_zero_context_gives_zeros():
    c = workloads.make_decode(3, 8, 2, 128, [5, 40, 600], 64, 16, torch.bfloat16, "cuda", 77)
    ctx = torch.tensor([0, 40, 0], dtype=torch.int64, device="cuda")
    out = ops.paged_decode(c.q, c.k_cache[0], c.v_cache[0], c.block_tables, ctx)
    torch.cuda.synchronize()
    assert out[0].eq(0).all() and out[2].eq(0).all()
    assert_attn_close(out[1], oracle_decode(c, seqs=[1])[1], torch.bfloat16, "ctx 40")


@pytest.mark.parametrize("heads", [16, 28])
def test_block_table_permutation_is_bit_invariant(heads):
    """Moving every block to another physical id (and updating the table) changes nothing
    (4 KV heads with groups of 4 and of 7, on the split kernel)."""
    c = workloads.make_decode(6, heads, 4, 128, [100, 700, 1600, 33, 512, 2049], 1024, 16,
                              torch.bfloat16, "cuda", 91)
    out1 = run_step(c)
    perm = torch.randperm(1024, generator=torch.Generator().manual_seed(1)).cuda()
    k2 = torch.empty_like(c.k_cache[0])
    v2 = torch.empty_like(c.v_cache[0])
    k2[perm] = c.k_cache[0]
    v2[perm] = c.v_cache[0]
    bt2 = perm[c.block_tables.long()].to(torch.int32)
    out2 = ops.paged_decode(c.q, k2, v2, bt2, c.context_lens)
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)


@pytest.mark.parametrize("heads", [8, 14])
def test_garbage_past_context_and_in_padding_blocks_is_ignored(heads):
    """NaN in slots past L (same block) and in block 0 (padded table entries), for groups
    of 4 and of 7."""
    c = workloads.make_decode(4, heads, 2, 128, [20, 33, 48, 100], 64, 16, torch.bfloat16,
                              "cuda", 5)
    out1 = run_step(c)
    kc, vc = c.k_cache[0], c.v_cache[0]
    used = {b for t in c.tables_list for b in t}
    for i, L in enumerate(c.lens):
        last = c.tables_list[i][(L - 1) // 16]
        kc[last, :, (L - 1) % 16 + 1:] = float("nan")
        vc[last, :, (L - 1) % 16 + 1:] = float("inf")
    if 0 not in used:
        kc[0] = float("nan")
        vc[0] = float("nan")
    out2 = ops.paged_decode(c.q, kc, vc, c.block_tables, c.context_lens)
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)


def test_closed_forms():
    """L = 1 gives v_0 exactly; equal keys give mean(V); constant V gives that constant."""
    hkv, g, d = 2, 4, 128
    c = workloads.make_decode(3, hkv * g, hkv, d, [1, 300, 300], 64, 16, torch.float32, "cuda", 8)
    kc, vc = c.k_cache[0], c.v_cache[0]
    # sequence 1: identical keys
    ids1 = c.tables_list[1]
    kc[ids1] = kc[ids1[0], :, :1].clone()  # broadcast key 0 to every slot of its blocks
    # sequence 2: constant values per head
    ids2 = c.tables_list[2]
    vc[ids2] = torch.arange(hkv, device="cuda", dtype=torch.float32).view(1, hkv, 1, 1) + 0.25
    out = ops.paged_decode(c.q, kc, vc, c.block_tables, c.context_lens)
    torch.cuda.synchronize()
    v0 = vc[c.tables_list[0][0], :, 0]  # (H_kv, D)
    assert torch.equal(out[0], v0.repeat_interleave(g, 0))
    vv = vc[torch.tensor(ids1, device="cuda")].permute(1, 0, 2, 3).reshape(hkv, -1, d)[:, :300]
    torch.testing.assert_close(out[1], vv.mean(1).repeat_interleave(g, 0), atol=1e-5, rtol=0)
    exp2 = (torch.arange(hkv, device="cuda", dtype=torch.float32) + 0.25).repeat_interleave(g)
    torch.testing.assert_close(out[2], exp2.view(-1, 1).expand(-1, d), atol=1e-6, rtol=0)


def test_gqa_equals_mha_with_repeated_kv():
    g, hkv = 4, 2
    c = workloads.make_decode(5, hkv * g, hkv, 128, [40, 90, 600, 1, 257], 128, 16,
                              torch.bfloat16, "cuda", 13)
    out_gqa = run_step(c)
    k_mha = c.k_cache[0].repeat_interleave(g, dim=1).contiguous()
    v_mha = c.v_cache[0].repeat_interleave(g, dim=1).contiguous()
    out_mha = ops.paged_decode(c.q, k_mha, v_mha, c.block_tables, c.context_lens)
    torch.cuda.synchronize()
    # Not bit-equal: a group shares its lazy-rescale decisions across its heads.
    assert_attn_close(out_gqa, out_mha.double().cpu().numpy(), torch.bfloat16, "GQA vs MHA")


def test_four_dim_query_and_explicit_scale():
    c = workloads.decode_small("cuda", torch.float32)
    run_step(c)
    out4 = ops.paged_decode(c.q.unsqueeze(1), c.k_cache[0], c.v_cache[0], c.block_tables,
                            c.context_lens, scale=0.05)
    torch.cuda.synchronize()
    assert out4.shape == (4, 1, 16, 128)
    assert_attn_close(out4[:, 0], oracle_decode(c, scale=0.05), torch.float32, "scale 0.05")


def test_query_layouts_and_the_output_layout_they_give():
    """The same queries in several layouts give bit-identical results: (B, H, D), (B, 1, H, D)
    (output (B, 1, H, D)), rows with gaps (output contiguous) and a head-major permutation
    (output in the same layout); a given `out` of either rank is filled in place."""
    c = workloads.make_decode(6, 16, 8, 128, [5, 70, 300, 1, 129, 64], 64, 16, torch.bfloat16,
                              "cuda", seed=31)
    ops.kv_write(c.k_new, c.v_new, c.k_cache[0], c.v_cache[0], c.slot_mapping)
    args = (c.k_cache[0], c.v_cache[0], c.block_tables, c.context_lens)
    base = ops.paged_decode(c.q, *args)
    out4 = ops.paged_decode(c.q.unsqueeze(1), *args)
    wide = torch.zeros(6, 16, 192, dtype=torch.bfloat16, device="cuda")
    wide[..., :128] = c.q
    gapped = ops.paged_decode(wide[..., :128], *args)
    head_major = c.q.transpose(0, 1).contiguous().transpose(0, 1)
    permuted = ops.paged_decode(head_major, *args)
    given3 = torch.empty_like(c.q)
    given4 = torch.empty(6, 1, 16, 128, dtype=torch.bfloat16, device="cuda")
    r3 = ops.paged_decode(c.q, *args, out=given3)
    r4 = ops.paged_decode(c.q.unsqueeze(1), *args, out=given4)
    torch.cuda.synchronize()
    assert base.shape == (6, 16, 128) and base.is_contiguous()
    assert out4.shape == (6, 1, 16, 128) and torch.equal(out4[:, 0], base)
    assert gapped.is_contiguous() and torch.equal(gapped, base)
    assert permuted.stride() == head_major.stride() and torch.equal(permuted, base)
    assert r3 is given3 and torch.equal(given3, base)
    assert r4 is given4 and torch.equal(given4[:, 0], base)
    assert_attn_close(base, oracle_decode(c), torch.bfloat16, "layouts")


def test_one_workspace_shared_by_every_path_and_a_graph():
    """One workspace shared by bf16 calls of several batch sizes (the LDS-indexed and the
    large-batch prologue), an fp32 call (whose partitions overwrite the partial region)
    and an fp8 call: every result equals the one computed with the cached workspace, and
    repeated calls are bit-identical.  Then the same call captured in a HIP graph and
    replayed three times, with eager calls on the same workspace in between."""
    lens = [int(x) for x in torch.randint(1, 4097, (48,),
                                          generator=torch.Generator().manual_seed(93))]
    a = workloads.make_decode(48, 32, 8, 128, lens, 16384, 16, torch.bfloat16, "cuda",
                              seed=93, max_blocks=256)
    big = workloads.make_decode(1100, 16, 4, 128, [1 + i % 60 for i in range(1100)], 8192, 16,
                                torch.bfloat16, "cuda", seed=94, max_blocks=4)
    f32 = workloads.decode_small("cuda", torch.float32)
    f8 = workloads.quantize_cache_fp8(a)
    need = max(ops.decode_workspace_bytes(c.batch, c.q.shape[1], c.num_kv_heads,
                                          c.block_tables.shape[1], 16, 128, c.q.dtype)
               for c in (a, big, f32))
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")

    def call(c, workspace, fp8=False):
        kw = dict(k_scale=f8.k_scale[0], v_scale=f8.v_scale[0]) if fp8 else {}
        kc, vc = (f8.k_cache[0], f8.v_cache[0]) if fp8 else (c.k_cache[0], c.v_cache[0])
        return ops.paged_decode(c.q, kc, vc, c.block_tables, c.context_lens,
                                workspace=workspace, **kw)

    expected = {}
    for name, c, fp8 in (("a", a, False), ("big", big, False), ("f32", f32, False),
                         ("fp8", a, True)):
        expected[name] = call(c, None, fp8)
    torch.cuda.synchronize()
    for name, c, fp8 in (("a", a, False), ("f32", f32, False), ("big", big, False),
                         ("fp8", a, True), ("a", a, False), ("a", a, False)):
        out = call(c, ws, fp8)
        torch.cuda.synchronize()
        assert torch.equal(out, expected[name]), name
    assert_attn_close(expected["a"], oracle_decode(a), torch.bfloat16, "shared workspace")

    out = torch.empty_like(a.q)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # warm-up off the capture
        ops.paged_decode(a.q, a.k_cache[0], a.v_cache[0], a.block_tables, a.context_lens,
                         out=out, workspace=ws)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.paged_decode(a.q, a.k_cache[0], a.v_cache[0], a.block_tables, a.context_lens,
                         out=out, workspace=ws)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, expected["a"])
        assert torch.equal(call(big, ws), expected["big"])  # eager work in between
        torch.cuda.synchronize()


def test_out_or_workspace_off_the_device_raises_before_launch():
    """A call whose plan is cached (same shapes and strides) but whose ``out`` or
    ``workspace`` lies on the host raises ValueError instead of handing the kernel a host
    pointer."""
    c = workloads.make_decode(3, 8, 2, 128, [5, 40, 600], 64, 16, torch.bfloat16, "cuda", 78)
    args = (c.q, c.k_cache[0], c.v_cache[0], c.block_tables, c.context_lens)
    good = ops.paged_decode(*args, out=torch.empty_like(c.q))
    with pytest.raises(ValueError, match="device"):
        ops.paged_decode(*args, out=torch.empty(c.q.shape, dtype=c.q.dtype))
    need = ops.decode_workspace_bytes(3, 8, 2, c.block_tables.shape[1], 16, 128)
    with pytest.raises(ValueError, match="workspace"):
        ops.paged_decode(*args, workspace=torch.empty(need, dtype=torch.uint8))
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    again = ops.paged_decode(*args, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(good, again)
