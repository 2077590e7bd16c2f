"""Drop-in layers end to end vs the reference pipeline restated on the CPU.

The GPU side is the package's PagedCausalSelfAttention / VisionAttention /
scaled_dot_product_attention in bf16.  The CPU side recomputes the same layer
in float64 from the same bf16 weights and inputs: projections, QK-RMSNorm and
RoPE as torch ops, then the oracle's op-for-op restatement of the reference's
attention (oracle.reference_attention, src/nano_inference/layers/attention.py:
267-332 and layers/vision.py:190-208).  Metadata comes from the oracle's
restatement of the reference's context builder.
Module-level bar (bf16 activations between every op on the GPU side):
max-abs <= 3e-2, mean-abs <= 3e-3.
"""
import pytest
import torch

from nano_inference_amd import (AttentionMetadata, PagedCausalSelfAttention, VisionAttention,
                                scaled_dot_product_attention)
from nano_inference_amd.layers import RMSNorm, RotaryEmbedding, rotate_half
from oracle import metadata as meta
from oracle import reference_attention as ref

pytestmark = pytest.mark.gpu

MOD_MAX_ABS = 3e-2
MOD_MEAN_ABS = 3e-3


def close(out, exp, what):
    d = (out.double().cpu() - exp.double().cpu()).abs()
    assert torch.isfinite(out).all(), what
    assert d.max().item() <= MOD_MAX_ABS and d.mean().item() <= MOD_MEAN_ABS, (
        f"{what}: max-abs {d.max().item():.3g}, mean-abs {d.mean().item():.3g}")


class CpuLayer:
    """The reference layer's math in float64 with the GPU module's weights."""

    def __init__(self, m: PagedCausalSelfAttention):
        sd = {k: v.detach().double().cpu() for k, v in m.state_dict().items()}
        self.m, self.sd = m, sd
        self.q_norm = self.k_norm = None
        if m.q_norm is not None:
            self.q_norm = RMSNorm(m.head_dim).double()
            self.q_norm.weight.data = sd["q_norm.weight"]
            self.k_norm = RMSNorm(m.head_dim).double()
            self.k_norm.weight.data = sd["k_norm.weight"]
        self.rot = RotaryEmbedding(m.head_dim, m.rotary.base)

    def forward(self, x, pos, mask, md, kc, vc, is_prefill):
        m, sd = self.m, self.sd
        b, s, _ = x.shape
        q = (x @ sd["q_proj.weight"].T).view(b, s, m.num_heads, m.head_dim)
        k = (x @ sd["k_proj.weight"].T).view(b, s, m.num_kv_heads, m.head_dim)
        v = (x @ sd["v_proj.weight"].T).view(b, s, m.num_kv_heads, m.head_dim)
        if self.q_norm is not None:
            q, k = self.q_norm(q), self.k_norm(k)
        q, k = self.rot(q, k, pos)
        attn = ref.paged_attention(q, k, v, kc, vc, md["slot_mapping"], md["kv_block_tables"],
                                   md["context_lens"], mask, is_prefill)
        return attn.reshape(b, s, -1) @ sd["o_proj.weight"].T


def test_paged_layer_prefill_then_decode_matches_reference_pipeline():
    torch.manual_seed(0)
    hidden, heads, kv, hd, bs, nb = 512, 4, 2, 128, 16, 64
    m = PagedCausalSelfAttention(hidden, heads, num_kv_heads=kv, head_dim=hd, use_qk_norm=True,
                                 rope_base=1e6).to("cuda", torch.bfloat16)
    m.layer_idx = 0
    cpu = CpuLayer(m)
    kc_g = torch.zeros((1, nb, kv, bs, hd), dtype=torch.bfloat16, device="cuda")
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
        out = m(x.cuda(), md["position_ids"].cuda(), md["attention_mask"].cuda(), mdg)
        exp = cpu.forward(x.double(), md["position_ids"], md["attention_mask"], md, kc_c, vc_c,
                          md["is_prefill"])
        return out, exp, md

    x = (torch.randn(3, max(prompts), hidden) * 0.5).to(torch.bfloat16)
    q_pf = [meta.Query(L, 0, meta.PREFILL, blocks[i], bs) for i, L in enumerate(prompts)]
    out, exp, md = step(q_pf, x)
    for i, L in enumerate(prompts):
        close(out[i, :L], exp[i, :L], f"prefill seq {i}")
    close(out, exp, "prefill incl. padded rows")
    # Bit-exact at the module level: the cache equals the reference's write loop
    # applied to the k/v the module itself produced on the GPU.
    with torch.no_grad():
        _, k_g, v_g, _ = m._qkv(x.cuda(), md["position_ids"].cuda(), None)
    kx = torch.zeros_like(kc_g[0]).cpu()
    vx = torch.zeros_like(vc_g[0]).cpu()
    ref.kv_write_loop(k_g.cpu(), v_g.cpu(), kx, vx, md["slot_mapping"])
    torch.cuda.synchronize()
    assert torch.equal(kc_g[0].cpu().view(torch.int16), kx.view(torch.int16)), "k cache bits"
    assert torch.equal(vc_g[0].cpu().view(torch.int16), vx.view(torch.int16)), "v cache bits"
    for t in range(1, 4):
        xd = (torch.randn(3, 1, hidden) * 0.5).to(torch.bfloat16)
        q_dec = [meta.Query(L, t, meta.DECODE, blocks[i], bs) for i, L in enumerate(prompts)]
        out, exp, _ = step(q_dec, xd)
        close(out, exp, f"decode step {t}")


def test_vision_attention_layer_matches_reference_pipeline():
    torch.manual_seed(1)
    hidden, heads = 160, 2  # head_dim 80, as the Qwen2.5-VL ViT
    m = VisionAttention(hidden, heads).to("cuda", torch.bfloat16)
    sd = {k: v.detach().double().cpu() for k, v in m.state_dict().items()}
    cu = torch.tensor([0, 64, 64 + 100, 64 + 100 + 37], dtype=torch.int32)
    t = int(cu[-1])
    x = (torch.randn(t, hidden) * 0.5).to(torch.bfloat16)
    ang = torch.randn(t, 40)
    emb = torch.cat([ang, ang], dim=-1)
    cos, sin = emb.cos(), emb.sin()
    out = m(x.cuda(), cu.cuda(), (cos.cuda(), sin.cuda()))
    xd = x.double()
    qkv = (xd @ sd["qkv.weight"].T + sd["qkv.bias"]).reshape(t, 3, heads, 80)
    q, k, v = qkv.permute(1, 0, 2, 3).unbind(0)
    c, s_ = cos.unsqueeze(1).double(), sin.unsqueeze(1).double()
    q, k = q * c + rotate_half(q) * s_, k * c + rotate_half(k) * s_
    a = ref.vision_attention(q, k, v, cu)
    exp = a @ sd["proj.weight"].T + sd["proj.bias"]
    close(out, exp, "vision layer")


def test_sdpa_free_function_with_prefix_mask():
    torch.manual_seed(2)
    b, h, hkv, s, d = 2, 4, 2, 70, 64
    q = torch.randn(b, h, s, d).to(torch.bfloat16)
    k = torch.randn(b, hkv, s, d).to(torch.bfloat16)
    v = torch.randn(b, hkv, s, d).to(torch.bfloat16)
    lens = torch.tensor([70, 41])
    mask2d = torch.arange(s).unsqueeze(0) < lens.unsqueeze(1)
    add = ref.additive_mask(mask2d, torch.float64)
    out = scaled_dot_product_attention(q.cuda(), k.cuda(), v.cuda(), add.cuda(), is_causal=True)
    kr = k.double().repeat_interleave(h // hkv, dim=1)
    vr = v.double().repeat_interleave(h // hkv, dim=1)
    exp = ref.sdpa(q.double(), kr, vr, attention_mask=add, is_causal=True)
    d_ = (out.double().cpu() - exp).abs()
    assert d_.max() <= 2e-2 and d_.mean() <= 2e-3, (d_.max(), d_.mean())
