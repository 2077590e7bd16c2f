"""Device context builder (nia_step_metadata) vs the oracle's restatement of the
reference's context builder: every tensor bit for bit.

Oracle: oracle.metadata.build_context, the loop-for-loop restatement of
src/nano_inference/engine/context_builder.py:83-193 and :18-81, pinned by the
reference's known answers (tests/test_context_builder_host.py).  Cases: those known
answers, seeded mixed prefill / recompute / decode batches at block sizes 4 and 16,
tables that end before the last position (the builder falls back to the last
block, as the reference does), mRoPE batches, one decode row, and a Qwen3-0.6B-generation-sized
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


def test_generation_sized_prefill_batch():
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


@pytest.mark.parametrize("seed", range(4))
def test_packed_layout_matches_padded_rows(seed):
    """nia_step_metadata_packed: row out_offset + j of every packed output equals
    column j of the padded oracle tensors; q_start / q_len / last_index describe the
    packing; a sequence with a device token index reads its token from there."""
    import numpy as np

    from nano_inference_amd import _lib

    qs = random_batch(300 + seed, 11, block_size=16 if seed % 2 else 4, short_tables=seed >= 2)
    exp = meta.build_context([to_oracle(q) for q in qs])
    steps = [exp["input_ids"][i, :int((exp["slot_mapping"][i] >= 0).sum())].tolist()
             for i in range(len(qs))]
    dev_tok = torch.arange(1000, 1100, dtype=torch.int64, device="cuda")
    hdr, toks, blks = [], [], []
    tok_off = blk_off = out_off = 0
    for i, (q, st) in enumerate(zip(qs, steps)):
        n = len(st)
        start = int(exp["position_ids"][i, 0])
        bl = q.kv_cache_block.block_ids
        src = 7 * i if n == 1 and i % 2 == 0 else -1  # some decodes read a device token
        hdr.append([n, start, len(bl), tok_off, blk_off, out_off, src, 0])
        if src < 0:
            toks += st
            tok_off += n
        blks += bl
        blk_off += len(bl)
        out_off += n
    b, t = len(qs), out_off
    desc = torch.tensor(np.concatenate([np.asarray(hdr, np.int64).reshape(-1),
                                        np.asarray(toks, np.int64), np.asarray(blks, np.int64)]),
                        device="cuda")
    mb = exp["kv_block_tables"].shape[1]
    i64 = dict(dtype=torch.int64, device="cuda")
    ids, pos, slots = (torch.full((t,), -7, **i64) for _ in range(3))
    ctx, last = torch.empty(b, **i64), torch.empty(b, **i64)
    qst = torch.empty(b, dtype=torch.int32, device="cuda")
    qln = torch.empty(b, dtype=torch.int32, device="cuda")
    tables = torch.empty((b, mb), dtype=torch.int32, device="cuda")
    rc = _lib.load().nia_step_metadata_packed(
        desc.data_ptr(), tok_off, blk_off, dev_tok.data_ptr(), dev_tok.numel(), b, t,
        max(len(s) for s in steps), mb, qs[0].kv_cache_block.block_size, ids.data_ptr(),
        pos.data_ptr(), slots.data_ptr(), ctx.data_ptr(), last.data_ptr(), qst.data_ptr(),
        qln.data_ptr(), tables.data_ptr(), None)
    assert rc == 0
    torch.cuda.synchronize()
    ids, pos, slots = ids.cpu(), pos.cpu(), slots.cpu()
    assert torch.equal(ctx.cpu(), exp["context_lens"])
    assert torch.equal(tables.cpu(), exp["kv_block_tables"])
    for i, (h, st) in enumerate(zip(hdr, steps)):
        n, o = h[0], h[5]
        want_ids = [1000 + h[6]] if h[6] >= 0 else st
        assert ids[o:o + n].tolist() == want_ids, i
        assert torch.equal(pos[o:o + n], exp["position_ids"][i, :n]), i
        assert torch.equal(slots[o:o + n], exp["slot_mapping"][i, :n]), i
        assert int(qst[i]) == o and int(qln[i]) == n and int(last[i]) == o + n - 1
