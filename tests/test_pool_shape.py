"""The one layout check of a paged KV pool (ops.check_pool_shape), run when the pool is
built (e2e.KVPool), against the limits every kernel the pool feeds declares in
include/nia_attn.h.  CPU only: nothing is launched."""
import pytest
import torch

from nano_inference_amd import e2e, ops


@pytest.mark.parametrize("bs", [4, 8, 16, 32, 64, 128, 256, 1024])
def test_power_of_two_block_sizes_pass_for_bf16(bs):
    ops.check_pool_shape(128, bs, 32, 8)
    ops.check_pool_shape(80, bs, 16, 16)


@pytest.mark.parametrize("bs", [1, 2, 3, 12, 24, 48, 100])
def test_other_bf16_block_sizes_are_refused(bs):
    with pytest.raises(ValueError, match="power-of-two block size"):
        ops.check_pool_shape(128, bs, 32, 8)


@pytest.mark.parametrize("bs,ok", [(16, True), (32, True), (256, True), (8, False),
                                   (48, False)])
def test_fp8_pools(bs, ok):
    if ok:
        ops.check_pool_shape(128, bs, 32, 8, torch.bfloat16, fp8_cache=True)
    else:
        with pytest.raises(ValueError, match="fp8"):
            ops.check_pool_shape(128, bs, 32, 8, torch.bfloat16, fp8_cache=True)
    with pytest.raises(ValueError, match="fp8"):
        ops.check_pool_shape(64, 16, 32, 8, torch.bfloat16, fp8_cache=True)


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
    with pytest.raises(ValueError, match="block size"):
        e2e.KVPool(cfg, 4, 24, torch.bfloat16, "cpu")
    with pytest.raises(ValueError, match="fp8"):
        e2e.KVPool(cfg, 4, 8, torch.bfloat16, "cpu", fp8=True)
