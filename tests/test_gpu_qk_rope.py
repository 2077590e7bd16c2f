"""Fused QK-RMSNorm + RoPE / mRoPE + KV write vs the oracle (oracle.qk_rope).

The oracle runs the reference's torch ops in the same order on CPU copies of the
same bf16 (or fp32) inputs (layers/norm.py:35-47, layers/rotary.py:8-33, :105-130,
:184-210).  Bar, bf16: at least 99.9% of q/k values bit-identical and every value
within 2^-6 of the oracle (the mean of squares is summed in another order, and
cos/sin come from another libm, so a value on a rounding boundary may move one
bf16 step); fp32: max-abs <= 1e-5.  The cache rows must be bit-identical to the
reference's write loop (attention.py:267-278) applied to the kernel's own k and
the input v.
"""
import pytest
import torch

from nano_inference_amd import ops
from nano_inference_amd._lib import NiaError
from oracle import qk_rope as O
from oracle import reference_attention as ref

pytestmark = pytest.mark.gpu

D = 128
EPS = 1e-6
MATCH_FRACTION = 0.999
BF16_MAX_ABS = 2.0 ** -6
F32_MAX_ABS = 1e-5


def _inputs(b, s, h, hkv, dtype, seed, norm=True, max_pos=40000):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, s, h, D, generator=g).to(dtype)
    k = torch.randn(b, s, hkv, D, generator=g).to(dtype)
    v = torch.randn(b, s, hkv, D, generator=g).to(dtype)
    qw = kw = None
    if norm:
        qw = (torch.randn(D, generator=g) * 0.3 + 1).to(dtype)
        kw = (torch.randn(D, generator=g) * 0.3 + 1).to(dtype)
    pos = torch.randint(0, max_pos, (b, s), generator=g)
    return q, k, v, qw, kw, pos


def _cuda(*ts):
    return [t.cuda() if t is not None else None for t in ts]


def _compare(out, exp, what):
    out, exp = out.cpu(), exp.cpu()
    assert torch.isfinite(out.float()).all(), what
    if out.dtype == torch.float32:
        d = (out - exp).abs().max().item()
        assert d <= F32_MAX_ABS, f"{what}: max-abs {d:.3g}"
        return
    same = (out.view(torch.int16) == exp.view(torch.int16)).float().mean().item()
    d = (out.float() - exp.float()).abs().max().item()
    assert same >= MATCH_FRACTION and d <= BF16_MAX_ABS, (
        f"{what}: {same:.5f} bit-identical, max-abs {d:.3g}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("norm", [True, False])
def test_rope_matches_oracle(dtype, norm):
    q, k, v, qw, kw, pos = _inputs(3, 37, 16, 8, dtype, seed=1 if norm else 2, norm=norm)
    freqs = O.inv_freq(D, 1e6)
    eq, ek = O.qk_norm_rope(q, k, qw, kw, EPS, pos, freqs)
    qg, kg, vg, qwg, kwg, pg = _cuda(q, k, v, qw, kw, pos)
    ops.qk_norm_rope_kv_write(qg, kg, vg, qwg, kwg, EPS, pg, freqs.cuda())
    _compare(qg, eq, "q")
    _compare(kg, ek, "k")
    assert torch.equal(vg.cpu(), v), "v must not change"


def test_mrope_image_positions_match_oracle():
    b, s, h, hkv = 2, 50, 16, 2
    q, k, v, qw, kw, _ = _inputs(b, s, h, hkv, torch.bfloat16, seed=3)
    g = torch.Generator().manual_seed(4)
    pos3 = torch.randint(0, 300, (3, b, s), generator=g)
    freqs = O.inv_freq(D, 1e6)
    sec = (16, 24, 24)
    eq, ek = O.qk_norm_rope(q, k, qw, kw, EPS, pos3, freqs, sec)
    qg, kg, vg, qwg, kwg, pg = _cuda(q, k, v, qw, kw, pos3)
    ops.qk_norm_rope_kv_write(qg, kg, vg, qwg, kwg, EPS, pg, freqs.cuda(), sec)
    _compare(qg, eq, "q")
    _compare(kg, ek, "k")


def test_cache_write_is_bit_exact_and_skips_padding():
    b, s, h, hkv, bs, nb = 4, 24, 16, 8, 16, 64
    q, k, v, qw, kw, pos = _inputs(b, s, h, hkv, torch.bfloat16, seed=5)
    g = torch.Generator().manual_seed(6)
    perm = torch.randperm(nb * bs, generator=g)[: b * s].view(b, s)
    slots = perm.clone()
    slots[1, 10:] = -1  # padding of a shorter sequence
    slots[3, 20:] = -1
    kc = torch.randn(nb, hkv, bs, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, hkv, bs, D, generator=g).to(torch.bfloat16)
    qg, kg, vg, qwg, kwg, pg, kcg, vcg, sg = _cuda(q, k, v, qw, kw, pos, kc, vc, slots)
    freqs = O.inv_freq(D, 1e6)
    ops.qk_norm_rope_kv_write(qg, kg, vg, qwg, kwg, EPS, pg, freqs.cuda(), None, kcg, vcg, sg)
    ek = O.qk_norm_rope(q, k, qw, kw, EPS, pos, freqs)[1]
    _compare(kg, ek, "k")
    kx, vx = kc.clone(), vc.clone()
    ref.kv_write_loop(kg.cpu(), v, kx, vx, slots)
    assert torch.equal(kcg.cpu().view(torch.int16), kx.view(torch.int16)), "k cache bits"
    assert torch.equal(vcg.cpu().view(torch.int16), vx.view(torch.int16)), "v cache bits"


def test_views_of_a_packed_qkv_projection():
    """q, k, v as column slices of one (tokens, (H + 2 H_kv) * D) projection output."""
    n, h, hkv = 77, 8, 2
    g = torch.Generator().manual_seed(8)
    qkv = torch.randn(n, (h + 2 * hkv) * D, generator=g).to(torch.bfloat16)
    qw = (torch.randn(D, generator=g) * 0.3 + 1).to(torch.bfloat16)
    kw = (torch.randn(D, generator=g) * 0.3 + 1).to(torch.bfloat16)
    pos = torch.arange(n) * 13
    freqs = O.inv_freq(D, 1e4)
    q, k, v = qkv.split([h * D, hkv * D, hkv * D], dim=-1)
    eq, ek = O.qk_norm_rope(q.reshape(1, n, h, D), k.reshape(1, n, hkv, D), qw, kw, EPS,
                            pos.view(1, n), freqs)
    qkv_g = qkv.cuda()
    qg, kg, vg = (t.view(n, -1, D) for t in qkv_g.split([h * D, hkv * D, hkv * D], dim=-1))
    ops.qk_norm_rope_kv_write(qg, kg, vg, qw.cuda(), kw.cuda(), EPS, pos.cuda(), freqs.cuda())
    _compare(qg.reshape(1, n, h, D), eq, "q")
    _compare(kg.reshape(1, n, hkv, D), ek, "k")
    assert torch.equal(qkv_g[:, (h + hkv) * D:].cpu(), qkv[:, (h + hkv) * D:]), "v untouched"


def test_layer_fused_path_equals_module_ops():
    """PagedCausalSelfAttention._qkv with and without the fused kernel."""
    from nano_inference_amd import PagedCausalSelfAttention
    torch.manual_seed(9)
    m = PagedCausalSelfAttention(512, 4, num_kv_heads=2, head_dim=D, use_qk_norm=True,
                                 rope_base=1e6).to("cuda", torch.bfloat16)
    x = (torch.randn(2, 33, 512, device="cuda") * 0.5).to(torch.bfloat16)
    pos = torch.arange(33, device="cuda").unsqueeze(0).expand(2, -1) + 100
    with torch.no_grad():
        m.fused_qk = True
        qf, kf, vf, _ = m._qkv(x, pos, None)
        m.fused_qk = False
        qt, kt, vt, _ = m._qkv(x, pos, None)
    _compare(qf, qt, "q")
    _compare(kf, kt, "k")
    assert torch.equal(vf, vt)


def test_unsupported_head_dim_raises():
    q = torch.zeros(4, 2, 64, device="cuda", dtype=torch.bfloat16)
    k = torch.zeros(4, 1, 64, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(NiaError):
        ops.qk_norm_rope_kv_write(q, k, k.clone(), None, None, 0.0,
                                  torch.zeros(4, dtype=torch.int64, device="cuda"),
                                  O.inv_freq(64, 1e4).cuda())
