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
    fields = list(AttentionMetadata.__dataclass_fields__)
    assert fields == ["context_lens", "kv_block_tables", "slot_mapping", "k_cache", "v_cache",
                      "is_prefill", "mrope_position_ids"]


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
