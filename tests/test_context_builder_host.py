"""Host side of the device context builder, and the oracle it is checked against (CPU).

- oracle.metadata.build_context against the reference's known answers
  (tests/unit/test_context_builder.py:14-58, :60-87: input_ids, positions, context
  lengths, tables, slots) and mRoPE invariants of the reference's own design
  (text rows equal the 1-D positions on every axis; a decode step's position equals
  the position a recompute of the same sequence gives that token).
- pack_queries: the descriptor, expanded here by a plain numpy reading of its
  documented layout, reproduces the oracle's tensors for seeded mixed batches; the
  GPU test checks the kernel's expansion of the same descriptor.
- The builder refuses a CPU device (there is no CPU path).
"""
import numpy as np
import pytest
import torch

from nano_inference_amd import GenerateContextBuilder
from nano_inference_amd.context_builder import HEADER_WORDS, pack_queries
from oracle import metadata as meta
from tests.queries import Stage, query, random_batch, to_oracle


def expand(pk):
    """Descriptor -> padded tensors, read off the documented layout."""
    d = pk.desc
    b, s = pk.batch, pk.max_step
    hdr = d[:b * HEADER_WORDS].reshape(b, HEADER_WORDS)
    tok = d[b * HEADER_WORDS:b * HEADER_WORDS + pk.num_tokens]
    blk = d[b * HEADER_WORDS + pk.num_tokens:b * HEADER_WORDS + pk.num_tokens + pk.num_blocks]
    mr = d[b * HEADER_WORDS + pk.num_tokens + pk.num_blocks:]
    assert mr.size == pk.num_mrope
    out = dict(input_ids=np.zeros((b, s), np.int64), position_ids=np.zeros((b, s), np.int64),
               slot_mapping=np.full((b, s), -1, np.int64), context_lens=np.zeros(b, np.int64),
               attention_mask=np.zeros((b, pk.max_total), bool),
               kv_block_tables=np.zeros((b, pk.max_blocks), np.int32),
               mrope=np.zeros((3, b, s), np.int64) if pk.has_mrope else None)
    bs = pk.block_size
    for i, (n, start, nb, to, bo, e, mo, c) in enumerate(hdr):
        out["context_lens"][i] = start + n
        out["attention_mask"][i, :start + n] = True
        out["kv_block_tables"][i, :nb] = blk[bo:bo + nb]
        for j in range(n):
            pos = start + j
            out["input_ids"][i, j] = tok[to + j]
            out["position_ids"][i, j] = pos
            bi = min(pos // bs, nb - 1)
            out["slot_mapping"][i, j] = blk[bo + bi] * bs + pos % bs
            if out["mrope"] is not None:
                for a in range(3):
                    out["mrope"][a, i, j] = mr[mo + a * e + j] if j < e else c + j - e
    return out


def check_against_oracle(queries):
    pk = pack_queries(queries)
    got = expand(pk)
    exp = meta.build_context([to_oracle(q) for q in queries])
    for k in ("input_ids", "position_ids", "slot_mapping", "context_lens", "attention_mask",
              "kv_block_tables"):
        assert np.array_equal(got[k], exp[k].numpy()), k
    if exp["mrope_position_ids"] is None:
        assert got["mrope"] is None
    else:
        assert np.array_equal(got["mrope"], exp["mrope_position_ids"].numpy())
    assert pk.is_prefill == exp["is_prefill"]


def test_oracle_known_answers_with_input_ids():
    c = meta.build_context([meta.FullQuery([1, 2, 3], [], meta.PREFILL, [101], 4),
                            meta.FullQuery([4, 5, 6, 7, 8], [], meta.PREFILL, [102, 103], 4)])
    assert c["input_ids"].tolist() == [[1, 2, 3, 0, 0], [4, 5, 6, 7, 8]]
    assert c["slot_mapping"][0, 0] == 404 and c["slot_mapping"][1, 4] == 412
    assert c["kv_block_tables"].tolist() == [[101, 0], [102, 103]]
    assert c["mrope_position_ids"] is None
    c = meta.build_context([meta.FullQuery([1, 2], [3, 4], meta.DECODE, [101], 16)])
    assert c["input_ids"].tolist() == [[4]] and c["position_ids"].tolist() == [[3]]
    assert c["context_lens"].tolist() == [4] and c["slot_mapping"].tolist() == [[1619]]


def test_oracle_mrope_invariants():
    plen, nout = 20, 5
    base = torch.arange(plen)
    mr = torch.stack([base // 4, base % 4, base + 50])
    prompt, outs = list(range(plen)), list(range(100, 100 + nout))
    text = meta.FullQuery(list(range(9)), [1, 2], meta.RECOMPUTE, [1], 16)
    vlm_rec = meta.FullQuery(prompt, outs, meta.RECOMPUTE, [2, 3], 16, mr)
    c = meta.build_context([text, vlm_rec])
    m = c["mrope_position_ids"]
    # text rows: every axis equals the 1-D positions over the step
    for a in range(3):
        assert torch.equal(m[a, 0, :11], c["position_ids"][0, :11])
    # a decode step after k outputs sees the position the recompute gives output k-1
    for k in range(1, nout + 1):
        dec = meta.FullQuery(prompt, outs[:k], meta.DECODE, [2, 3], 16, mr)
        cd = meta.build_context([dec])["mrope_position_ids"]
        assert all(int(cd[a, 0, 0]) == int(m[a, 1, plen + k - 1]) for a in range(3))
    # prompt columns are the explicit table
    assert torch.equal(m[:, 1, :plen], mr)


def test_packing_reproduces_the_oracle_known_answers():
    qs = [query([1, 2, 3], [], Stage.PREFILL, [101], 4, rid="q1"),
          query([4, 5, 6, 7, 8], [], Stage.PREFILL, [102, 103], 4, rid="q2")]
    check_against_oracle(qs)
    check_against_oracle([query([1, 2], [3, 4], Stage.DECODE, [101], 16)])
    check_against_oracle([query([1, 2, 3], [9, 8], Stage.RECOMPUTE, [7, 9], 4)])


@pytest.mark.parametrize("seed", range(6))
def test_packing_reproduces_the_oracle_on_mixed_batches(seed):
    check_against_oracle(random_batch(seed, 9, block_size=16 if seed % 2 else 4,
                                      short_tables=seed >= 3))


@pytest.mark.parametrize("seed", range(4))
def test_packing_reproduces_the_oracle_mrope(seed):
    check_against_oracle(random_batch(100 + seed, 7, mrope=True))


def test_packing_errors():
    with pytest.raises(ValueError):
        pack_queries([])
    mr = torch.zeros(3, 4, dtype=torch.int64)
    qs = [query([1, 2, 3, 4], [], Stage.PREFILL, [1], 16, mr),
          query([5, 6], [], Stage.PREFILL, [2], 16)]  # text prefill in an mRoPE batch
    with pytest.raises(ValueError):
        pack_queries(qs)
    with pytest.raises(ValueError):  # mRoPE table shorter than the prompt
        pack_queries([query([1] * 9, [], Stage.PREFILL, [1], 16, torch.zeros(3, 4))])


def test_builder_has_no_cpu_path():
    with pytest.raises(ValueError):
        GenerateContextBuilder(torch.device("cpu"))
