"""Host-side memo of results that read a tensor back (ops.TensorMemo), as used for the
prefix-mask check of the layers (and the general additive path other masks take) and the
max chunk length of varlen attention: one
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


def test_non_prefix_masks_go_to_the_general_path():
    """A mask that is not a prefix gives no key lengths (None, memoised too), and the
    additive form the reference adds to the scores (attention.py:40-47) is built for it:
    a 2-D bool mask as 0 / -inf, a float mask cast to the scores' dtype, broadcastable."""
    cpu = torch.device("cpu")
    bad = torch.tensor([[1, 0, 1, 0]], dtype=torch.bool)
    for _ in range(2):
        assert A._prefix_lengths(bad, 1, 4, cpu) is None
    assert A._prefix_lengths(torch.ones(1, 2, 1, 4), 1, 4, cpu) is None
    soft = torch.zeros(1, 1, 1, 4)
    soft[0, 0, 0, 1] = -2.5  # finite, non-zero: an additive bias, not a visibility mask
    assert A._prefix_lengths(soft, 1, 4, cpu) is None
    add = A._additive_mask(bad, 1, 3, 2, 4, torch.bfloat16)
    assert add.shape == (1, 1, 1, 4) and add.dtype == torch.bfloat16
    assert add[0, 0, 0].tolist() == [0.0, float("-inf"), 0.0, float("-inf")]
    wide = torch.randn(2, 3, 5, 7)
    got = A._additive_mask(wide, 2, 3, 5, 6, torch.float32)  # sliced to S_k = 6
    assert torch.equal(got, wide[..., :6])
    with pytest.raises(ValueError, match="broadcast"):
        A._additive_mask(torch.zeros(2, 4, 5, 6), 2, 3, 5, 6, torch.float32)


def test_mask_operand_alignment_and_broadcast_strides():
    """ops._mask_operand: fp32, rows whose strides are multiples of four elements (a copy
    with keys padded to four when needed), and stride 0 for broadcast dimensions."""
    m = torch.randn(1, 3, 1, 6)  # 6 keys: rows of 6 floats are not 16-byte multiples
    op, st = ops._mask_operand(m, 2, 3, 5, 6, torch.device("cpu"))
    assert op.dtype == torch.float32 and op.shape[-1] == 8 and st[0] == 0 and st[2] == 0
    assert st[1] % 4 == 0 and torch.equal(op[..., :6], m)
    op2, st2 = ops._mask_operand(torch.zeros(2, 1, 4, 8), 2, 5, 4, 8, torch.device("cpu"))
    assert st2 == (32, 0, 8) and op2.shape == (2, 1, 4, 8)
    with pytest.raises(ValueError):
        ops._mask_operand(torch.zeros(3, 1, 4, 8), 2, 5, 4, 8, torch.device("cpu"))


def test_mask_operand_covers_the_rows_and_keys_the_kernels_read():
    """A mask with fewer rows than the longest query run or fewer keys than the longest key
    run raises (the kernels would read past it); size-1 row and key dimensions broadcast,
    the key dimension materialised (the kernels read a mask row's keys as a row)."""
    cpu = torch.device("cpu")
    with pytest.raises(ValueError, match="rows"):
        ops._mask_operand(torch.zeros(1, 1, 4, 8), 1, 2, 5, 8, cpu)
    with pytest.raises(ValueError, match="keys"):
        ops._mask_operand(torch.zeros(1, 1, 5, 8), 1, 2, 5, 9, cpu)
    m = torch.randn(2, 1, 1, 1)
    op, st = ops._mask_operand(m, 2, 3, 5, 7, cpu)
    assert op.shape == (2, 1, 1, 8) and st[1] == 0 and st[2] == 0 and st[0] % 4 == 0
    assert torch.equal(op[..., :7], m.expand(2, 1, 1, 7))
    # longer masks are fine (the kernels read a prefix of every row)
    op3, _ = ops._mask_operand(torch.zeros(1, 2, 9, 12), 1, 2, 5, 8, cpu)
    assert op3.shape == (1, 2, 9, 12)


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
