"""nia_paged_decode_noalloc (decode with the library's fixed scratch array) through the
C ABI against nia_paged_decode with a caller workspace: two calls in a row, the second
with a smaller batch, each bit-identical to the workspace entry point and within the
bf16 bar of the float64 oracle.  The first call on the device also clears the array."""
import ctypes
import math

import pytest
import torch

from nano_inference_amd import _lib, ops, workloads
from oracle import textbook as tb
from tests.tolerances import assert_attn_close

pytestmark = pytest.mark.gpu


def _noalloc(c, out):
    lib = _lib.load()
    q = c.q
    b, h, d = q.shape
    nb, hkv, bs, _ = c.k_cache[0].shape
    st = lib.nia_paged_decode_noalloc(
        out.data_ptr(), out.stride(0), out.stride(1), q.data_ptr(), q.stride(0), q.stride(1),
        c.k_cache[0].data_ptr(), c.v_cache[0].data_ptr(), c.block_tables.data_ptr(),
        c.block_tables.stride(0), c.block_tables.shape[1], c.context_lens.data_ptr(), b, h, hkv,
        d, bs, nb, 1.0 / math.sqrt(d), _lib.DTYPE_BF16,
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check("nia_paged_decode_noalloc", st)


def _oracle(c):
    return tb.paged_decode(c.q.double().cpu().numpy(), c.k_cache[0].double().cpu().numpy(),
                           c.v_cache[0].double().cpu().numpy(), c.block_tables.cpu().numpy(),
                           c.context_lens.cpu().numpy(), 1.0 / math.sqrt(c.q.shape[2]))


def test_noalloc_decode_matches_workspace_decode_twice():
    big = workloads.make_decode(48, 32, 8, 128, [int(x) for x in torch.randint(
        1, 4097, (48,), generator=torch.Generator().manual_seed(61))], 8192, 16,
        torch.bfloat16, "cuda", seed=61, max_blocks=256)
    small = workloads.make_decode(5, 28, 4, 128, [1, 17, 300, 2049, 700], 1024, 16,
                                  torch.bfloat16, "cuda", seed=62)
    for c in (big, small):
        ops.kv_write(c.k_new, c.v_new, c.k_cache[0], c.v_cache[0], c.slot_mapping)
        exp = ops.paged_decode(c.q, c.k_cache[0], c.v_cache[0], c.block_tables, c.context_lens)
        out = torch.empty_like(c.q)
        _noalloc(c, out)
        torch.cuda.synchronize()
        assert torch.equal(out, exp), f"batch {c.batch}: differs from nia_paged_decode"
        assert_attn_close(out, _oracle(c), torch.bfloat16, f"noalloc batch {c.batch}")
