"""The E2E generator's step metadata vs the oracle's restatement of the reference
context builder (src/nano_inference/engine/context_builder.py:83-193), on the CPU:
slots, block tables and context lengths equal; the prefill mask is the builder's
prefix mask and the prefill positions agree on every real token.
"""
import torch

from nano_inference_amd import e2e
from oracle import metadata as meta


def _gen(block_size=16):
    cfg = e2e.Qwen3Config(num_layers=1)
    pool = e2e.KVPool(cfg, 64, block_size, torch.float32, torch.device("cpu"))
    return e2e.Generator(None, pool, max_new_tokens=5)


def test_prefill_metadata_matches_context_builder():
    gen = _gen()
    prompts = [[1] * n for n in (5, 33, 16, 1)]
    seqs = [e2e._Seq(p, gen.pool.allocate(len(p) + 5)) for p in prompts]
    ids, pos, valid, md, last = gen._prefill_inputs(seqs)
    ref = meta.build([meta.Query(len(p), 0, meta.PREFILL, s.blocks, 16)
                      for p, s in zip(prompts, seqs)])
    assert torch.equal(md.slot_mapping, ref["slot_mapping"])
    assert torch.equal(md.kv_block_tables, ref["kv_block_tables"])
    assert torch.equal(md.context_lens, ref["context_lens"])
    assert torch.equal(valid, ref["attention_mask"])
    assert torch.equal(pos[valid], ref["position_ids"][valid])
    assert torch.equal(last, torch.tensor([n - 1 for n in (5, 33, 16, 1)]))
    assert md.is_prefill


def test_decode_metadata_matches_context_builder():
    gen = _gen()
    prompts = [[2] * n for n in (5, 31, 16, 47)]
    seqs = [e2e._Seq(p, gen.pool.allocate(len(p) + 5)) for p in prompts]
    gen._bt = gen._tables(seqs)
    gen._lens = torch.tensor([len(p) for p in prompts], dtype=torch.int64)
    gen._rows = torch.arange(len(seqs))
    for step in range(1, 5):
        gen._step = torch.tensor([step], dtype=torch.int64)
        p, slot, ctx = gen._decode_positions()
        ref = meta.build([meta.Query(len(pr), step, meta.DECODE, s.blocks, 16)
                          for pr, s in zip(prompts, seqs)])
        assert torch.equal(slot.unsqueeze(1), ref["slot_mapping"])
        assert torch.equal(ctx, ref["context_lens"])
        assert torch.equal(p.unsqueeze(1), ref["position_ids"])
        assert torch.equal(gen._bt, ref["kv_block_tables"])


def test_generation_prompts_are_seeded():
    a = e2e.generation_prompts(8, 128, 2048, seed=4004)
    b = e2e.generation_prompts(8, 128, 2048, seed=4004)
    assert a == b
    assert all(128 <= len(p) <= 2048 for p in a)
    assert all(0 <= t < 151936 for p in a for t in p)
