"""Host-side memo of results that read a tensor back (ops.TensorMemo), as used for the
prefix-mask check of the layers and the max chunk length of varlen attention: one
device read per tensor, recomputed when the tensor is modified in place, never reused
for another tensor.  Runs on the CPU (the memo and the mask check are device-agnostic).
"""
import pytest
import torch

from nano_inference_amd import attention as A
from nano_inference_amd import ops


def test_memo_hits_only_the_same_unmodified_tensor():
    memo = ops.TensorMemo(size=2)
    a = torch.zeros(4)
    b = torch.zeros(4)
    memo.put(a, "k", 1)
    assert memo.get(a, "k") == 1
    assert memo.get(a, "other") is None
    assert memo.get(b, "k") is None  # equal contents, another tensor
    a.add_(1)  # in place: version counter moves
    assert memo.get(a, "k") is None
    memo.put(a, "k", 2)
    memo.put(b, "k", 3)
    c = torch.zeros(1)
    memo.put(c, "k", 4)  # evicts the oldest entry (size 2)
    assert memo.get(a, "k") is None and memo.get(b, "k") == 3 and memo.get(c, "k") == 4


def test_prefix_lengths_checked_once_per_mask():
    cpu = torch.device("cpu")
    mask = torch.tensor([[1, 1, 1, 0], [1, 1, 0, 0]], dtype=torch.bool)
    lens = A._prefix_lengths(mask, 2, 4, cpu)
    assert lens.tolist() == [3, 2] and lens.dtype == torch.int32
    assert A._prefix_lengths(mask, 2, 4, cpu) is lens  # memo hit: no second read
    additive = torch.zeros(2, 1, 1, 4)
    additive[0, 0, 0, 3:] = float("-inf")
    assert A._prefix_lengths(additive, 2, 4, cpu).tolist() == [3, 4]
    mask[1, 2] = True  # modified in place: checked again
    assert A._prefix_lengths(mask, 2, 4, cpu).tolist() == [3, 3]


def test_non_prefix_masks_still_raise_every_time():
    cpu = torch.device("cpu")
    bad = torch.tensor([[1, 0, 1, 0]], dtype=torch.bool)
    for _ in range(2):
        with pytest.raises(NotImplementedError, match="prefix"):
            A._prefix_lengths(bad, 1, 4, cpu)
    with pytest.raises(NotImplementedError, match="shape"):
        A._prefix_lengths(torch.ones(1, 2, 1, 4), 1, 4, cpu)


def test_varlen_max_seqlen_memo():
    cu = torch.tensor([0, 5, 12, 13], dtype=torch.int32)
    ops._MAX_SEQLEN.put(cu, "max", 7)
    assert ops._MAX_SEQLEN.get(cu, "max") == 7
    cu[1] = 6
    assert ops._MAX_SEQLEN.get(cu, "max") is None


def test_rope_table_converted_once_per_table_and_again_after_a_change():
    table = (1.0 / 10000 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128)).to(
        torch.bfloat16)
    first = ops._inv_freq_f32(table)
    assert first.dtype == torch.float32 and first.is_contiguous()
    assert torch.equal(first, table.float())
    assert ops._inv_freq_f32(table) is first          # the same table: no new conversion
    table.mul_(2)                                      # an in-place change: converted again
    again = ops._inv_freq_f32(table)
    assert again is not first and torch.equal(again, table.float())
    other = table.clone()                              # another tensor with equal values
    assert ops._inv_freq_f32(other) is not again


def test_rope_tables_of_every_layer_stay_converted():
    """A model holds one table per layer; all of them stay in the memo."""
    tables = [torch.full((64,), 1.0 + i, dtype=torch.bfloat16) for i in range(64)]
    first = [ops._inv_freq_f32(t) for t in tables]
    assert all(ops._inv_freq_f32(t) is f for t, f in zip(tables, first))
