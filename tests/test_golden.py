"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every fixture and the seeded inputs still
hash to the stored digest (so a GPU mismatch is never generator drift).
GPU: the kernels on the same seeded inputs match the fixtures to the parity bar.
"""
import os

import numpy as np
import pytest
import torch

from nano_inference_amd import ops, workloads
from tests.golden import make_golden as mg
from tests.tolerances import assert_attn_close

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(HERE, f"{name}.npz"), allow_pickle=False) as z:
        return str(z["digest"]), z["out"].astype(np.float64)


@pytest.mark.parametrize("name", sorted(mg.FIXTURES))
def test_oracle_reproduces_fixture(name):
    dig, out = mg.FIXTURES[name]()
    fdig, fout = load(name)
    assert dig == fdig, "seeded inputs changed"
    np.testing.assert_array_equal(out.astype(np.float32), fout.astype(np.float32))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_kernel_matches_fixture(dtype):
    c = workloads.decode_small("cpu", dtype)
    _, fout = load("decode_small_f32" if dtype == torch.float32 else "decode_small_bf16")
    g = lambda t: t.cuda()  # noqa: E731
    kc, vc = g(c.k_cache[0]), g(c.v_cache[0])
    ops.kv_write(g(c.k_new), g(c.v_new), kc, vc, g(c.slot_mapping))
    out = ops.paged_decode(g(c.q), kc, vc, g(c.block_tables), g(c.context_lens))
    torch.cuda.synchronize()
    assert_attn_close(out, fout, dtype, "golden decode")


@pytest.mark.gpu
def test_varlen_kernels_match_fixtures():
    c = workloads.make_varlen([3, 17, 40], 4, 2, 128, torch.bfloat16, "cpu", 606, True)
    out = ops.varlen_attention(c.q.cuda(), c.k.cuda(), c.v.cuda(), c.cu_seqlens.cuda(),
                               causal=True)
    torch.cuda.synchronize()
    assert_attn_close(out, load("varlen_causal_small")[1], torch.bfloat16, "golden varlen")
    from nano_inference_amd.vision import window_index
    cu = window_index([(1, 8, 12)])[1]
    lens = [int(b - a) for a, b in zip(cu[:-1], cu[1:])]
    v = workloads.make_varlen(lens, 2, 2, 80, torch.bfloat16, "cpu", 707, False)
    outv = ops.varlen_attention(v.q.cuda(), v.k.cuda(), v.v.cuda(), v.cu_seqlens.cuda())
    torch.cuda.synchronize()
    assert_attn_close(outv, load("vision_window_small")[1], torch.bfloat16, "golden vision")


@pytest.mark.gpu
def test_chunked_kernel_matches_fixture():
    c = workloads.chunked_qwen3_8b("cpu", n=2, chunk=24, prior=[40, 3], seed=808, num_heads=4,
                                   num_kv_heads=2)
    out = ops.prefill_paged(c.q.cuda(), c.k_cache.cuda(), c.v_cache.cuda(),
                            c.block_tables.cuda(), c.q_start.cuda(), c.q_len.cuda(),
                            c.context_lens.cuda(), c.chunk)
    torch.cuda.synchronize()
    assert_attn_close(out, load("chunked_small")[1], torch.bfloat16, "golden chunked")
