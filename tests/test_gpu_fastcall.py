"""The two routes to the library give the same results on the GPU: every hot op run through
the CPython fast-call module and through the ctypes binding (the route taken where the
module has not been built) writes bit-identical outputs and caches."""
import pytest
import torch

from nano_inference_amd import _lib, ops, workloads

pytestmark = pytest.mark.gpu


def _through(route):
    """Point _lib.calls() at `route` ("fast" or "ctypes")."""
    lib = _lib.load()
    if route == "fast":
        _lib._calls = None  # rebinds _nia_fast on the next call
        assert _lib.calls() is not lib, "_nia_fast is not built"
    else:
        _lib._calls, _lib._calls_lib = lib, lib
        assert _lib.calls() is lib


def _run_all():
    torch.manual_seed(0)
    out = {}
    # KV write (bf16 and fp8) into fresh pools
    c = workloads.make_decode(6, 16, 8, 128, [5, 70, 300, 1, 129, 64], 64, 16, torch.bfloat16,
                              "cuda", seed=41)
    kc, vc = torch.zeros_like(c.k_cache[0]), torch.zeros_like(c.v_cache[0])
    ops.kv_write(c.k_new, c.v_new, kc, vc, c.slot_mapping)
    out["kv_write"] = (kc.clone(), vc.clone())
    k8 = torch.zeros(kc.shape, dtype=torch.uint8, device="cuda")
    v8 = torch.zeros_like(k8)
    ks = torch.zeros(kc.shape[:3], dtype=torch.float32, device="cuda")
    vs = torch.zeros_like(ks)
    ops.kv_write(c.k_new, c.v_new, k8, v8, c.slot_mapping, ks, vs)
    out["kv_write_fp8"] = (k8.clone(), v8.clone(), ks.clone(), vs.clone())
    # decode, bf16 and over the fp8 pool just written
    ops.kv_write(c.k_new, c.v_new, c.k_cache[0], c.v_cache[0], c.slot_mapping)
    out["decode"] = ops.paged_decode(c.q, c.k_cache[0], c.v_cache[0], c.block_tables,
                                     c.context_lens)
    out["decode_fp8"] = ops.paged_decode(c.q, k8, v8, c.block_tables, c.context_lens,
                                         k_scale=ks, v_scale=vs)
    # prefill (contiguous) and chunked prefill over the paged cache
    r = workloads.make_varlen([1, 33, 200, 257], 16, 4, 128, torch.bfloat16, "cuda", seed=42,
                              causal=True)
    cu = r.cu_seqlens
    qs, ql = cu[:-1].contiguous(), (cu[1:] - cu[:-1]).contiguous()
    out["prefill"] = ops.prefill(r.q, r.k, r.v, qs, ql, qs, ql, max(r.lens),
                                 ops.CAUSAL_TOP_LEFT)
    ch = workloads.chunked_qwen3_8b("cuda", n=3, chunk=64, prior=[0, 100, 333])
    out["prefill_paged"] = ops.prefill_paged(ch.q, ch.k_cache, ch.v_cache, ch.block_tables,
                                             ch.q_start, ch.q_len, ch.context_lens, ch.chunk)
    # fused QK-norm + RoPE + KV write, in place on copies of one input
    g = torch.Generator().manual_seed(43)
    q = torch.randn(4, 1, 16, 128, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(4, 1, 8, 128, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(4, 1, 8, 128, generator=g).to(torch.bfloat16).cuda()
    w = (torch.randn(128, generator=g) * 0.3 + 1).to(torch.bfloat16).cuda()
    pos = torch.randint(0, 4000, (4, 1), generator=g).cuda()
    inv = (1.0 / 1e6 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128)).cuda()
    kq, vq = torch.zeros_like(c.k_cache[0]), torch.zeros_like(c.v_cache[0])
    slots = torch.arange(4, dtype=torch.int64, device="cuda").reshape(4, 1) * 3
    ops.qk_norm_rope_kv_write(q, k, v, w, w, 1e-6, pos, inv, None, kq, vq, slots)
    out["qk"] = (q, k, kq, vq)
    torch.cuda.synchronize()
    return out


def test_fast_calls_and_ctypes_give_identical_results():
    saved = (_lib._calls, _lib._calls_lib)
    try:
        _through("ctypes")
        ref = _run_all()
        _through("fast")
        got = _run_all()
    finally:
        _lib._calls, _lib._calls_lib = saved
    for name in ref:
        a, b = ref[name], got[name]
        a = a if isinstance(a, tuple) else (a,)
        b = b if isinstance(b, tuple) else (b,)
        for x, y in zip(a, b):
            assert torch.equal(x, y), name
