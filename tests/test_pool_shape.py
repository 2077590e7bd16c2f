"""The one layout check of a paged KV pool (ops.check_pool_shape), run when the pool is
built (e2e.KVPool), against the limits every kernel the pool feeds declares in
include/nia_attn.h.  CPU only: nothing is launched."""
import pytest
import torch

from nano_inference_amd import e2e, ops


@pytest.mark.parametrize("bs", [1, 2, 3, 4, 8, 12, 16, 24, 48, 100, 256, 1024])
def test_bf16_pools_take_any_block_size(bs):
    """The reference's block size is any positive integer (src/nano_inference/core/
    config.py:54); sizes the tuned kernels do not take run the any-size kernel."""
    ops.check_pool_shape(128, bs, 32, 8)
    ops.check_pool_shape(80, bs, 16, 16)


@pytest.mark.parametrize("bs", [0, -16])
def test_block_sizes_must_be_positive(bs):
    with pytest.raises(ValueError, match="positive"):
        ops.check_pool_shape(128, bs, 32, 8)


@pytest.mark.parametrize("bs", [1, 8, 12, 16, 32, 48, 256])
def test_fp8_pools(bs):
    ops.check_pool_shape(128, bs, 32, 8, torch.bfloat16, fp8_cache=True)
    with pytest.raises(ValueError, match="fp8"):
        ops.check_pool_shape(64, bs, 32, 8, torch.bfloat16, fp8_cache=True)


def test_fp32_takes_any_block_size_and_every_group():
    for bs in (1, 3, 12, 16, 48):
        ops.check_pool_shape(96, bs, 64, 2, torch.float32)


def test_groups_and_head_dims():
    ops.check_pool_shape(128, 16, 64, 1)  # 64 query heads on one KV head
    with pytest.raises(ValueError, match="divisible"):
        ops.check_pool_shape(128, 16, 30, 8)
    with pytest.raises(ValueError, match="head_dim"):
        ops.check_pool_shape(112, 16, 32, 8)


def test_pool_construction_checks_its_layout():
    cfg = e2e.Qwen3Config(num_layers=1)
    e2e.KVPool(cfg, 4, 128, torch.bfloat16, "cpu")
    e2e.KVPool(cfg, 4, 24, torch.bfloat16, "cpu")
    e2e.KVPool(cfg, 4, 8, torch.bfloat16, "cpu", fp8=True)
    with pytest.raises(ValueError, match="positive"):
        e2e.KVPool(cfg, 4, 0, torch.bfloat16, "cpu")
    with pytest.raises(ValueError, match="head_dim"):
        e2e.KVPool(e2e.Qwen3Config(num_layers=1, head_dim=112), 4, 16, torch.bfloat16, "cpu")
