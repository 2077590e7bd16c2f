"""Pins of oracle.reference_attention, the torch-CPU restatement of the reference (CPU).

Checked against torch.nn.functional.scaled_dot_product_attention (a library
routine independent of both), against the float64 textbook, and against the
invariants the reference's own tests state (tests/unit/test_attention.py:16-33).
The restatement keeps the reference's fp32 softmax even for float64 inputs
(src/nano_inference/layers/attention.py:49), so float64 comparisons use a
2e-6 bar - a wrong term, index or scale shows up at O(1e-2) or more.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import metadata as meta
from oracle import reference_attention as ref
from oracle import textbook as tb
from oracle import vision_windows as vw

SOFTMAX_F32 = 2e-6


def g(seed):
    return torch.Generator().manual_seed(seed)


@pytest.mark.parametrize("causal", [True, False])
def test_sdpa_matches_library_routine(causal):
    q = torch.randn(2, 4, 9, 16, generator=g(1), dtype=torch.float64)
    k = torch.randn(2, 4, 9, 16, generator=g(2), dtype=torch.float64)
    v = torch.randn(2, 4, 9, 16, generator=g(3), dtype=torch.float64)
    ours = ref.sdpa(q, k, v, is_causal=causal)
    lib = F.scaled_dot_product_attention(q, k, v, is_causal=causal)
    torch.testing.assert_close(ours, lib, atol=SOFTMAX_F32, rtol=0)


def test_sdpa_padding_mask_matches_library_and_textbook():
    lens = torch.tensor([9, 5])
    mask2d = torch.arange(9).unsqueeze(0) < lens.unsqueeze(1)
    q = torch.randn(2, 4, 9, 16, generator=g(4), dtype=torch.float64)
    k = torch.randn(2, 4, 9, 16, generator=g(5), dtype=torch.float64)
    v = torch.randn(2, 4, 9, 16, generator=g(6), dtype=torch.float64)
    ours = ref.sdpa(q, k, v, attention_mask=ref.additive_mask(mask2d, q.dtype), is_causal=True)
    tri = torch.ones(9, 9, dtype=torch.bool).tril()
    lib_mask = tri.unsqueeze(0) & mask2d.unsqueeze(1)
    lib = F.scaled_dot_product_attention(q, k, v, attn_mask=lib_mask.unsqueeze(1))
    torch.testing.assert_close(ours, lib, atol=SOFTMAX_F32, rtol=0)
    for b in range(2):
        for h in range(4):
            bnd = np.minimum(np.arange(9) + 1, int(lens[b]))
            exp = tb.attend(q[b, h].numpy(), k[b, h].numpy(), v[b, h].numpy(), 0.25, bnd)
            np.testing.assert_allclose(ours[b, h].numpy(), exp, atol=SOFTMAX_F32)


def test_sdpa_no_causal_mask_when_lengths_differ():
    """Quirk of the reference (attention.py:33-38): S_q != S_k means no triu."""
    q = torch.randn(1, 2, 3, 8, generator=g(7), dtype=torch.float64)
    k = torch.randn(1, 2, 5, 8, generator=g(8), dtype=torch.float64)
    v = torch.randn(1, 2, 5, 8, generator=g(9), dtype=torch.float64)
    torch.testing.assert_close(ref.sdpa(q, k, v, is_causal=True), ref.sdpa(q, k, v, is_causal=False))


def _decode_setup(dtype=torch.float64):
    bs, nb, hkv, h, d = 4, 32, 2, 4, 8
    lens = [5, 12, 1]
    perm = torch.randperm(nb, generator=g(10)).tolist()
    queries, off = [], 0
    for L in lens:
        n = -(-L // bs)
        queries.append(meta.Query(L - 1, 1, meta.DECODE, perm[off:off + n], bs))
        off += n
    md = meta.build(queries)
    kc = torch.randn(nb, hkv, bs, d, generator=g(11), dtype=dtype)
    vc = torch.randn(nb, hkv, bs, d, generator=g(12), dtype=dtype)
    q = torch.randn(3, 1, h, d, generator=g(13), dtype=dtype)
    kn = torch.randn(3, 1, hkv, d, generator=g(14), dtype=dtype)
    vn = torch.randn(3, 1, hkv, d, generator=g(15), dtype=dtype)
    return md, kc, vc, q, kn, vn


def test_paged_decode_restatement_matches_textbook():
    md, kc, vc, q, kn, vn = _decode_setup()
    out = ref.paged_attention(q, kn, vn, kc, vc, md["slot_mapping"], md["kv_block_tables"],
                              md["context_lens"], md["attention_mask"], is_prefill=False)
    exp = tb.paged_decode(q[:, 0].numpy(), kc.numpy(), vc.numpy(), md["kv_block_tables"].numpy(),
                          md["context_lens"].numpy(), 1 / math.sqrt(8))
    np.testing.assert_allclose(out[:, 0].numpy(), exp, atol=SOFTMAX_F32)


def test_paged_decode_finite_garbage_in_padding_is_masked():
    md, kc, vc, q, kn, vn = _decode_setup()
    args = (md["slot_mapping"], md["kv_block_tables"], md["context_lens"], md["attention_mask"])
    out1 = ref.paged_attention(q, kn, vn, kc.clone(), vc.clone(), *args, is_prefill=False)
    used = set(md["kv_block_tables"][0].tolist()) | set(md["kv_block_tables"][1].tolist())
    kc2, vc2 = kc.clone(), vc.clone()
    for b in range(kc.shape[0]):
        if b not in used:
            kc2[b], vc2[b] = 1e4, -1e4
    out2 = ref.paged_attention(q, kn, vn, kc2, vc2, *args, is_prefill=False)
    torch.testing.assert_close(out1, out2, atol=0, rtol=0)


def test_kv_write_loop_closed_form_and_negative_slots():
    bs, nb, hkv, d = 4, 8, 2, 3
    kc = torch.zeros(nb, hkv, bs, d)
    vc = torch.zeros(nb, hkv, bs, d)
    k = torch.arange(2 * 3 * hkv * d, dtype=torch.float32).view(2, 3, hkv, d)
    slots = torch.tensor([[9, -1, 31], [0, 4, -1]])
    ref.kv_write_loop(k, -k, kc, vc, slots)
    for b in range(2):
        for s in range(3):
            sl = int(slots[b, s])
            if sl >= 0:
                assert torch.equal(kc[sl // bs, :, sl % bs], k[b, s])
                assert torch.equal(vc[sl // bs, :, sl % bs], -k[b, s])
    assert int((kc != 0).any(dim=(1, 3)).sum()) == 4  # four (block, offset) rows touched


def test_prefill_causality_invariant():
    """Mirror of tests/unit/test_attention.py:16-33 on the restated prefill path."""
    b, s, h, d = 1, 6, 2, 8
    q = torch.randn(b, s, h, d, generator=g(20))
    k = torch.randn(b, s, h, d, generator=g(21))
    v = torch.randn(b, s, h, d, generator=g(22))
    kc = torch.zeros(4, h, 4, d)
    slots = torch.full((b, s), -1)
    mask = torch.ones(b, s, dtype=torch.bool)
    bt = torch.zeros(b, 2, dtype=torch.int32)
    ctx = torch.tensor([s])
    o1 = ref.paged_attention(q, k, v, kc, kc.clone(), slots, bt, ctx, mask, True)
    k2, v2 = k.clone(), v.clone()
    k2[:, 3:] = torch.randn(b, 3, h, d, generator=g(23))
    v2[:, 3:] = torch.randn(b, 3, h, d, generator=g(24))
    o2 = ref.paged_attention(q, k2, v2, kc, kc.clone(), slots, bt, ctx, mask, True)
    torch.testing.assert_close(o1[:, :3], o2[:, :3], atol=1e-5, rtol=1e-5)


def test_padded_prefill_rows_equal_packed_rows():
    lens = [7, 3]
    s, h, d = 7, 2, 8
    q = torch.randn(2, s, h, d, generator=g(30), dtype=torch.float64)
    k = torch.randn(2, s, h, d, generator=g(31), dtype=torch.float64)
    v = torch.randn(2, s, h, d, generator=g(32), dtype=torch.float64)
    mask = torch.arange(s).unsqueeze(0) < torch.tensor(lens).unsqueeze(1)
    out = ref.paged_attention(q, k, v, torch.zeros(1, h, 4, d, dtype=torch.float64),
                              torch.zeros(1, h, 4, d, dtype=torch.float64),
                              torch.full((2, s), -1), torch.zeros(2, 1, dtype=torch.int32),
                              torch.tensor(lens), mask, True)
    for i, L in enumerate(lens):
        packed = tb.varlen(q[i].numpy(), k[i].numpy(), v[i].numpy(), [0], [L], [0], [L],
                           1 / math.sqrt(d), "top_left")[0][1]
        np.testing.assert_allclose(out[i, :L].numpy(), packed, atol=SOFTMAX_F32)
        # padded rows (past L) attend to every valid key, as the reference's mask gives
        pad = tb.varlen(q[i].numpy(), k[i].numpy(), v[i].numpy(), [0], [s], [0], [L],
                        1 / math.sqrt(d), "top_left")[0][1]
        np.testing.assert_allclose(out[i].numpy(), pad, atol=SOFTMAX_F32)


def test_vision_restatement_matches_textbook_and_is_chunk_order_invariant():
    grids = [(1, 4, 8), (1, 8, 8)]
    cu = vw.full_cu_seqlens(grids)
    t = int(cu[-1])
    q = torch.randn(t, 2, 8, generator=g(40), dtype=torch.float64)
    k = torch.randn(t, 2, 8, generator=g(41), dtype=torch.float64)
    v = torch.randn(t, 2, 8, generator=g(42), dtype=torch.float64)
    out = ref.vision_attention(q, k, v, cu).view(t, 2, 8)
    res = tb.varlen(q.numpy(), k.numpy(), v.numpy(), cu[:-1].numpy(), np.diff(cu.numpy()),
                    cu[:-1].numpy(), np.diff(cu.numpy()), 1 / math.sqrt(8), "none")
    for s, (idx, o) in res.items():
        np.testing.assert_allclose(out[int(cu[s]) + idx].numpy(), o, atol=SOFTMAX_F32)
    # swap the two images in the packing: per-image outputs are unchanged
    n0 = int(cu[1])
    sw = [torch.cat([x[n0:], x[:n0]]) for x in (q, k, v)]
    cu2 = torch.tensor([0, t - n0, t], dtype=torch.int32)
    out2 = ref.vision_attention(*sw, cu2).view(t, 2, 8)
    torch.testing.assert_close(out2[t - n0:], out[:n0], atol=SOFTMAX_F32, rtol=0)
