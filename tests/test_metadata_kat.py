"""The oracle's context-builder restatement against the reference's known answers.

Known answers from tests/unit/test_context_builder.py:14-58 (prefill batch) and
:60-87 (decode step) of the reference.
"""
import torch

from oracle import metadata as meta


def test_prefill_batch_known_answers():
    md = meta.build([meta.Query(3, 0, meta.PREFILL, [101], 4),
                     meta.Query(5, 0, meta.PREFILL, [102, 103], 4)])
    assert md["is_prefill"]
    assert md["position_ids"].shape == (2, 5) and md["attention_mask"].shape == (2, 5)
    assert torch.equal(md["context_lens"], torch.tensor([3, 5]))
    assert torch.equal(md["kv_block_tables"], torch.tensor([[101, 0], [102, 103]],
                                                           dtype=torch.int32))
    sm = md["slot_mapping"]
    assert sm[0, 0] == 404 and sm[0, 2] == 406 and sm[1, 0] == 408 and sm[1, 4] == 412
    assert sm[0, 3] == -1 and sm[0, 4] == -1  # padding
    assert md["kv_block_tables"].dtype == torch.int32 and sm.dtype == torch.int64


def test_decode_step_known_answers():
    md = meta.build([meta.Query(2, 2, meta.DECODE, [101], 16)])
    assert not md["is_prefill"]
    assert md["position_ids"][0, 0] == 3
    assert md["context_lens"][0] == 4
    assert md["slot_mapping"][0, 0] == 1619
    assert md["attention_mask"].tolist() == [[True] * 4]


def test_recompute_refeeds_prompt_and_outputs_from_zero():
    md = meta.build([meta.Query(3, 2, meta.RECOMPUTE, [7, 9], 4)])
    assert md["position_ids"].tolist() == [[0, 1, 2, 3, 4]]
    assert md["slot_mapping"].tolist() == [[28, 29, 30, 31, 36]]
