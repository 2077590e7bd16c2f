"""General additive attention masks through the drop-in scaled_dot_product_attention and
the dense (no-cache) layer path: masks that are not prefixes go to nia_prefill_masked,
which adds them to the scaled scores as src/nano_inference/layers/attention.py:40-47
does (any mask broadcastable to (B, H, S_q, S_k), sliced to S_k, cast to the scores'
dtype), with the causal triu of :33-38 when S_q == S_k.

Oracle: float64 numpy, softmax(q k^T / sqrt(D) [+ triu] + mask) v per (batch, head), the
mask taken at the scores' dtype as the reference casts it; oracle.reference_attention.sdpa
(the reference's op order) cross-checks one case.  Rows with every key masked are zeros
(the reference's softmax gives NaN).  Bars: bf16 max-abs 2e-2 / mean-abs 2e-3, fp32 1e-5.
"""
import math

import numpy as np
import pytest
import torch

from nano_inference_amd import ops, scaled_dot_product_attention
from oracle import reference_attention as ref
from tests.tolerances import assert_attn_close

pytestmark = pytest.mark.gpu


def oracle(q, k, v, mask4, causal):
    """q (B, H, Sq, D), k/v (B, Hkv, Sk, D), mask4 broadcastable (B, H, Sq, Sk) float64."""
    q, k, v = (t.double().cpu().numpy() for t in (q, k, v))
    b, h, sq, d = q.shape
    sk = k.shape[2]
    g = h // k.shape[1]
    m = np.broadcast_to(mask4.double().cpu().numpy(), (b, h, sq, sk))
    out = np.zeros((b, h, sq, d))
    tri = np.triu(np.ones((sq, sk), dtype=bool), 1) if causal and sq == sk else None
    for i in range(b):
        for j in range(h):
            s = q[i, j] @ k[i, j // g].T / math.sqrt(d) + m[i, j]
            if tri is not None:
                s = np.where(tri, -np.inf, s)
            mx = s.max(axis=1, keepdims=True)
            ok = np.isfinite(mx[:, 0])
            p = np.exp(s - np.where(np.isfinite(mx), mx, 0.0))
            den = p.sum(axis=1, keepdims=True)
            out[i, j][ok] = (p[ok] @ v[i, j // g]) / den[ok]
    return out


def inputs(b, h, hkv, sq, sk, d, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn((b, h, sq, d), generator=g, device="cuda").to(dtype)
    k = torch.randn((b, hkv, sk, d), generator=g, device="cuda").to(dtype)
    v = torch.randn((b, hkv, sk, d), generator=g, device="cuda").to(dtype)
    return q, k, v


def holes(shape, frac, seed):
    """-inf at a fraction of positions, else N(0, 2^2) (an additive bias, not a prefix)."""
    g = torch.Generator().manual_seed(seed)
    m = torch.randn(shape, generator=g) * 2.0
    m[torch.rand(shape, generator=g) < frac] = float("-inf")
    return m


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", ["full", "per_key", "per_head", "rows_only"])
def test_sdpa_additive_masks(dtype, shape):
    b, h, hkv, s, d = 2, 8, 2, 150, 128
    q, k, v = inputs(b, h, hkv, s, s, d, dtype, 11)
    mshape = {"full": (b, h, s, s), "per_key": (b, 1, 1, s), "per_head": (1, h, s, s),
              "rows_only": (s, s)}[shape]
    mask = holes(mshape, 0.2, 12).cuda()
    out = scaled_dot_product_attention(q, k, v, attention_mask=mask, is_causal=True)
    torch.cuda.synchronize()
    m4 = mask.to(dtype).double()  # the reference casts the mask to the scores' dtype
    while m4.dim() < 4:
        m4 = m4.unsqueeze(0)
    assert_attn_close(out, oracle(q, k, v, m4, True), dtype, f"{shape} mask {dtype}")


def test_sdpa_mask_longer_than_keys_is_sliced_and_non_causal_rows():
    """S_q != S_k (no triu) and a (B, 1, 1, S_total) mask wider than S_k; one row's keys
    all masked gives zeros."""
    b, h, sq, sk, d = 3, 4, 5, 77, 128
    q, k, v = inputs(b, h, h, sq, sk, d, torch.bfloat16, 21)
    mask = holes((b, 1, sq, sk + 9), 0.3, 22)
    mask[1, 0, 2, :] = float("-inf")
    mask = mask.cuda()
    out = scaled_dot_product_attention(q, k, v, attention_mask=mask, is_causal=True)
    torch.cuda.synchronize()
    assert out[1, :, 2].eq(0).all()
    exp = oracle(q, k, v, mask[..., :sk].to(torch.bfloat16).double(), False)
    assert_attn_close(out, exp, torch.bfloat16, "wide mask")


@pytest.mark.parametrize("d", [64, 80, 96])
def test_sdpa_masks_other_head_dims(d):
    b, h, s = 2, 4, 97
    q, k, v = inputs(b, h, h, s, s, d, torch.bfloat16, 30 + d)
    mask = holes((b, 1, s, s), 0.1, 31).cuda()
    out = scaled_dot_product_attention(q, k, v, attention_mask=mask, is_causal=False)
    torch.cuda.synchronize()
    exp = oracle(q, k, v, mask.to(torch.bfloat16).double(), False)
    assert_attn_close(out, exp, torch.bfloat16, f"D={d} mask")


def test_sdpa_mask_matches_the_reference_op_order():
    """The restated reference sdpa (float64 inputs, its own cast points) on the same mask."""
    b, h, s, d = 1, 4, 64, 128
    q, k, v = inputs(b, h, h, s, s, d, torch.float32, 41)
    mask = holes((b, h, s, s), 0.15, 42).cuda()
    out = scaled_dot_product_attention(q, k, v, attention_mask=mask, is_causal=True)
    exp = ref.sdpa(q.double().cpu(), k.double().cpu(), v.double().cpu(),
                   attention_mask=mask.double().cpu(), is_causal=True)
    torch.cuda.synchronize()
    e = exp.numpy()
    o = out.double().cpu().numpy()
    nan_rows = np.isnan(e).any(axis=-1)  # every key masked: NaN in the reference, 0 here
    assert (o[nan_rows] == 0).all()
    # the restatement's softmax runs in fp32, as the reference's
    assert_attn_close(o[~nan_rows], e[~nan_rows], torch.float32, "reference op order")


def test_prefix_masks_still_take_the_key_length_path():
    """A prefix mask is turned into key lengths (no mask operand): same result as the
    general path on the same mask (bf16 bar), through ops.prefill directly."""
    b, h, s, d = 2, 4, 80, 128
    q, k, v = inputs(b, h, h, s, s, d, torch.bfloat16, 51)
    lens = torch.tensor([80, 33])
    m2 = torch.arange(s).unsqueeze(0) < lens.unsqueeze(1)
    add = ref.additive_mask(m2, torch.bfloat16).cuda()
    out_prefix = scaled_dot_product_attention(q, k, v, attention_mask=add, is_causal=True)
    q3 = q.transpose(1, 2).reshape(b * s, h, d)
    k3 = k.transpose(1, 2).reshape(b * s, h, d)
    v3 = v.transpose(1, 2).reshape(b * s, h, d)
    st = torch.arange(b, dtype=torch.int32, device="cuda") * s
    ln = torch.full((b,), s, dtype=torch.int32, device="cuda")
    out_mask = ops.prefill(q3, k3, v3, st, ln, st, ln, s, ops.CAUSAL_TOP_LEFT,
                           mask=add.float())
    torch.cuda.synchronize()
    assert_attn_close(out_prefix, oracle(q, k, v, add.double(), True), torch.bfloat16, "prefix")
    assert_attn_close(out_mask.view(b, s, h, d).transpose(1, 2),
                      oracle(q, k, v, add.double(), True), torch.bfloat16, "as a mask")


def test_varlen_masks_cover_rows_and_keys_or_raise():
    """ops.prefill with a mask over ragged sequences: a mask with fewer keys than the longest
    sequence's, or fewer rows than the longest query run, raises ValueError before any launch
    (the kernels would read past it); a key-broadcast mask ([S, 1, rows, 1], one bias per
    query row) gives the unmasked attention, since softmax ignores a per-row constant."""
    lens = [5, 9]
    t = sum(lens)
    g = torch.Generator(device="cuda").manual_seed(77)
    q = torch.randn((t, 2, 64), generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn((t, 2, 64), generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn((t, 2, 64), generator=g, device="cuda").to(torch.bfloat16)
    st = torch.tensor([0, 5], dtype=torch.int32, device="cuda")
    ln = torch.tensor(lens, dtype=torch.int32, device="cuda")
    args = (q, k, v, st, ln, st, ln, 9, ops.CAUSAL_NONE)
    with pytest.raises(ValueError, match="keys"):
        ops.prefill(*args, mask=torch.zeros(2, 1, 9, 8, device="cuda"))
    with pytest.raises(ValueError, match="rows"):
        ops.prefill(*args, mask=torch.zeros(2, 1, 8, 9, device="cuda"))
    plain = ops.prefill(*args)
    per_row = torch.randn(2, 1, 9, 1, generator=g, device="cuda")
    got = ops.prefill(*args, mask=per_row)
    torch.cuda.synchronize()
    assert (got.float() - plain.float()).abs().max().item() < 2e-2
