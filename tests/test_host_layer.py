"""Host-side layer behaviour that needs no GPU: validation and interface parity (CPU)."""
import pytest
import torch

from nano_inference_amd import (AttentionMetadata, PagedCausalSelfAttention,
                                Qwen25VLDecoderAttention, VisionAttention, ops)


def test_constructor_validation_matches_reference_messages():
    with pytest.raises(ValueError, match="hidden_size must be divisible by num_heads"):
        PagedCausalSelfAttention(30, 4)
    with pytest.raises(ValueError, match="num_heads must be divisible by num_kv_heads"):
        PagedCausalSelfAttention(32, 4, num_kv_heads=3)


def test_parameter_names_match_reference_layer():
    m = PagedCausalSelfAttention(64, 4, num_kv_heads=2, head_dim=32, use_qk_norm=True)
    names = set(m.state_dict())
    assert names == {"q_proj.weight", "k_proj.weight", "v_proj.weight", "o_proj.weight",
                     "q_norm.weight", "k_norm.weight"}
    assert m.q_proj.out_features == 128 and m.k_proj.out_features == 64
    assert m.layer_idx is None
    vl = Qwen25VLDecoderAttention(64, 4, num_kv_heads=2, head_dim=32, mrope_section=(4, 6, 6))
    assert set(vl.state_dict()) == {"q_proj.weight", "k_proj.weight", "v_proj.weight",
                                    "o_proj.weight"}
    va = VisionAttention(1280, 16)
    assert va.head_dim == 80 and set(va.state_dict()) == {"qkv.weight", "qkv.bias",
                                                         "proj.weight", "proj.bias"}


def test_metadata_fields_match_reference_dataclass():
    """The reference's fields in its order (core/context.py:7-24); the only additions are
    the optional fp8 row scales and the caller-owned decode workspace, after them and
    defaulting to None."""
    fields = AttentionMetadata.__dataclass_fields__
    assert list(fields)[:7] == ["context_lens", "kv_block_tables", "slot_mapping", "k_cache",
                                "v_cache", "is_prefill", "mrope_position_ids"]
    assert list(fields)[7:] == ["k_scale", "v_scale", "decode_workspace"]
    assert all(fields[f].default is None for f in ("k_scale", "v_scale", "decode_workspace"))


def test_ops_refuse_cpu_tensors():
    q = torch.zeros(2, 4, 128)
    kc = torch.zeros(4, 2, 16, 128)
    bt = torch.zeros(2, 1, dtype=torch.int32)
    ctx = torch.ones(2, dtype=torch.int64)
    with pytest.raises(ValueError, match="GPU only"):
        ops.paged_decode(q, kc, kc, bt, ctx)
    with pytest.raises(ValueError, match="GPU only"):
        ops.kv_write(q.view(2, 1, 4, 128)[:, :, :2], q.view(2, 1, 4, 128)[:, :, :2], kc, kc,
                     torch.zeros(2, 1, dtype=torch.int64))


def test_mrope_with_equal_axes_is_1d_rope():
    """Mirror of the reference's tests/unit/test_mrope.py:21-40 on the package layers."""
    from nano_inference_amd.layers import MRotaryEmbedding, RotaryEmbedding

    torch.manual_seed(0)
    q = torch.randn(2, 5, 4, 128)
    k = torch.randn(2, 5, 2, 128)
    pos = torch.arange(5).unsqueeze(0).expand(2, -1) + 7
    a = RotaryEmbedding(128, 1e6)(q, k, pos)
    b = MRotaryEmbedding(128, 1e6, (16, 24, 24))(q, k, pos.unsqueeze(0).expand(3, -1, -1))
    torch.testing.assert_close(a[0], b[0], atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(a[1], b[1], atol=1e-5, rtol=1e-5)


def test_rmsnorm_formula():
    """RMSNorm = x / sqrt(mean(x^2) + eps) * w, fp32 inside (reference norm.py:35-47)."""
    from nano_inference_amd.layers import RMSNorm

    x = torch.randn(3, 7, 16, dtype=torch.float64)
    n = RMSNorm(16, eps=1e-6).double()
    n.weight.data = torch.linspace(0.5, 1.5, 16, dtype=torch.float64)
    exp = x / torch.sqrt((x ** 2).mean(-1, keepdim=True) + 1e-6) * n.weight
    torch.testing.assert_close(n(x), exp.to(x.dtype), atol=1e-6, rtol=1e-6)
