"""Device context builder (nia_step_metadata) vs the oracle's restatement of the
reference's context builder: every tensor bit for bit.

Oracle: oracle.metadata.build_context, the loop-for-loop restatement of
src/nano_inference/engine/context_builder.py:83-193 and :18-81, pinned by the
reference's known answers (tests/test_context_builder_host.py).  Cases: those known
answers, seeded mixed prefill / recompute / decode batches at block sizes 4 and 16,
tables that end before the last position (the builder falls back to the last
block, as the reference does), mRoPE batches, one decode row, and a config-4-sized
prefill batch (8 prompts up to 2048 tokens).
"""
import pytest
import torch

from nano_inference_amd import GenerateContextBuilder, select_last_logits
from oracle import metadata as meta
from tests.queries import Stage, query, random_batch, to_oracle

pytestmark = pytest.mark.gpu


def check(queries):
    ctx = GenerateContextBuilder(torch.device("cuda")).build(queries)
    exp = meta.build_context([to_oracle(q) for q in queries])
    md = ctx.metadata
    pairs = [("input_ids", ctx.input_ids), ("position_ids", ctx.position_ids),
             ("attention_mask", ctx.attention_mask), ("context_lens", md.context_lens),
             ("kv_block_tables", md.kv_block_tables), ("slot_mapping", md.slot_mapping)]
    for name, got in pairs:
        e = exp[name]
        assert got.dtype == e.dtype and got.shape == e.shape, (name, got.dtype, got.shape)
        assert torch.equal(got.cpu(), e), name
    if exp["mrope_position_ids"] is None:
        assert md.mrope_position_ids is None
    else:
        assert torch.equal(md.mrope_position_ids.cpu(), exp["mrope_position_ids"])
    assert md.is_prefill == exp["is_prefill"]
    assert ctx.request_ids == exp["request_ids"]
    assert ctx.token_histories == exp["token_histories"]
    steps = torch.tensor([len(q.generation_inputs.prompt_token_ids) if q.stage == Stage.PREFILL
                          else (len(q.generation_inputs.prompt_token_ids) +
                                len(q.output_token_ids) if q.stage == Stage.RECOMPUTE else 1)
                          for q in queries])
    assert torch.equal(ctx.last_token_index.cpu(), steps - 1)
    return ctx


def test_known_answers():
    check([query([1, 2, 3], [], Stage.PREFILL, [101], 4, rid="q1"),
           query([4, 5, 6, 7, 8], [], Stage.PREFILL, [102, 103], 4, rid="q2")])
    check([query([1, 2], [3, 4], Stage.DECODE, [101], 16)])
    check([query([1, 2, 3], [9, 8], Stage.RECOMPUTE, [7, 9], 4)])


@pytest.mark.parametrize("seed", range(8))
def test_mixed_batches(seed):
    check(random_batch(seed, 13, block_size=16 if seed % 2 else 4, short_tables=seed >= 4))


@pytest.mark.parametrize("seed", range(4))
def test_mrope_batches(seed):
    check(random_batch(200 + seed, 9, mrope=True))


def test_config4_prefill_batch():
    g = torch.Generator().manual_seed(4004)
    qs = []
    perm = torch.randperm(40000, generator=g).tolist()
    off = 0
    for i in range(8):
        n = int(torch.randint(128, 2049, (1,), generator=g))
        nb = -(-(n + 256) // 16)
        qs.append(query(torch.randint(0, 151936, (n,), generator=g).tolist(), [],
                        Stage.PREFILL, perm[off:off + nb], 16, rid=f"p{i}"))
        off += nb
    check(qs)


def test_last_token_select():
    qs = [query([5] * 7, [], Stage.PREFILL, [1], 16), query([6] * 3, [], Stage.PREFILL, [2], 16)]
    ctx = check(qs)
    logits = torch.arange(2 * 7 * 4, dtype=torch.float32, device="cuda").view(2, 7, 4)
    sel = select_last_logits(logits, ctx)
    assert torch.equal(sel.cpu(), torch.stack([logits[0, 6], logits[1, 2]]).cpu())
