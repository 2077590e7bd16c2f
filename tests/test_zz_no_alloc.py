"""nia_paged_decode_noalloc (decode with the library's fixed scratch array) through the
C ABI against nia_paged_decode with a caller workspace: two calls in a row, the second
with a smaller batch, each bit-identical to the workspace entry point and within the
bar of the float64 oracle.  Cases cover every path that uses the shared array: bf16
with the unit prefix built in LDS (batch <= 1024), bf16 with the prefix written to the
array by decode_prefix_kernel (batch 1100), the largest bf16 partial rows (16 query
heads per KV head at head_dim 128), and the fp32 partition kernel.  Nothing in the
array is cleared between calls: each call writes what it reads."""
import ctypes
import math

import pytest
import torch

from nano_inference_amd import _lib, ops, workloads
from oracle import textbook as tb
from tests.tolerances import assert_attn_close

pytestmark = pytest.mark.gpu


def _noalloc(c, out, dtype):
    lib = _lib.load()
    q = c.q
    b, h, d = q.shape
    nb, hkv, bs, _ = c.k_cache[0].shape
    code = _lib.DTYPE_BF16 if dtype == torch.bfloat16 else _lib.DTYPE_F32
    st = lib.nia_paged_decode_noalloc(
        out.data_ptr(), out.stride(0), out.stride(1), q.data_ptr(), q.stride(0), q.stride(1),
        c.k_cache[0].data_ptr(), c.v_cache[0].data_ptr(), c.block_tables.data_ptr(),
        c.block_tables.stride(0), c.block_tables.shape[1], c.context_lens.data_ptr(), b, h, hkv,
        d, bs, nb, 1.0 / math.sqrt(d), code,
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check("nia_paged_decode_noalloc", st)


def _oracle(c):
    return tb.paged_decode(c.q.double().cpu().numpy(), c.k_cache[0].double().cpu().numpy(),
                           c.v_cache[0].double().cpu().numpy(), c.block_tables.cpu().numpy(),
                           c.context_lens.cpu().numpy(), 1.0 / math.sqrt(c.q.shape[2]))


def _lens(n, hi, seed):
    return [int(x) for x in torch.randint(1, hi + 1, (n,),
                                          generator=torch.Generator().manual_seed(seed))]


def _check_pair(cases, dtype):
    for c in cases:
        ops.kv_write(c.k_new, c.v_new, c.k_cache[0], c.v_cache[0], c.slot_mapping)
        exp = ops.paged_decode(c.q, c.k_cache[0], c.v_cache[0], c.block_tables, c.context_lens)
        out = torch.empty_like(c.q)
        _noalloc(c, out, dtype)
        torch.cuda.synchronize()
        assert torch.equal(out, exp), f"batch {c.batch}: differs from nia_paged_decode"
        assert_attn_close(out, _oracle(c), dtype, f"noalloc {dtype} batch {c.batch}")


def test_noalloc_decode_matches_workspace_decode_twice():
    big = workloads.make_decode(48, 32, 8, 128, _lens(48, 4096, 61), 8192, 16,
                                torch.bfloat16, "cuda", seed=61, max_blocks=256)
    small = workloads.make_decode(5, 28, 4, 128, [1, 17, 300, 2049, 700], 1024, 16,
                                  torch.bfloat16, "cuda", seed=62)
    _check_pair((big, small), torch.bfloat16)


def test_noalloc_decode_prefix_kernel_batch_and_largest_group():
    """Batch 1100 (the unit prefix goes through the array), then 16 query heads per KV
    head at head_dim 128 (the largest partial rows) on a smaller batch."""
    wide = workloads.make_decode(1100, 8, 2, 128, _lens(1100, 40, 63), 4096, 16,
                                 torch.bfloat16, "cuda", seed=63, max_blocks=4)
    g16 = workloads.make_decode(7, 32, 2, 128, [3, 64, 900, 4000, 1, 2500, 17], 2048, 16,
                                torch.bfloat16, "cuda", seed=64)
    _check_pair((wide, g16), torch.bfloat16)


def test_noalloc_decode_fp32_partitions_twice():
    big = workloads.make_decode(12, 16, 8, 128, _lens(12, 3000, 65), 4096, 16, torch.float32,
                                "cuda", seed=65)
    small = workloads.make_decode(3, 16, 8, 128, [17, 511, 64], 128, 16, torch.float32, "cuda",
                                  seed=66)
    _check_pair((big, small), torch.float32)
