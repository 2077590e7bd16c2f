"""KV-cache write kernel vs the reference's per-token loop: bit-exact.

Oracle: oracle.reference_attention.kv_write_loop, the restatement of
src/nano_inference/layers/attention.py:267-278, run on CPU copies of the same
tensors.  Every byte of the cache is compared, so untouched slots are checked
too.
"""
import pytest
import torch

from nano_inference_amd import ops, workloads
from oracle import metadata as meta
from oracle import reference_attention as ref

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.detach().contiguous().cpu().view(torch.uint8)


def _check(k, v, k_cache, v_cache, slots):
    kr, vr = k_cache.cpu().clone(), v_cache.cpu().clone()
    ref.kv_write_loop(k.cpu(), v.cpu(), kr, vr, slots.cpu())
    ops.kv_write(k, v, k_cache, v_cache, slots)
    torch.cuda.synchronize()
    assert torch.equal(_bits(k_cache), _bits(kr))
    assert torch.equal(_bits(v_cache), _bits(vr))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_small_new_tokens(dtype):
    c = workloads.decode_small("cuda", dtype)
    _check(c.k_new, c.v_new, c.k_cache[0], c.v_cache[0], c.slot_mapping)


def test_decode_qwen3_8b_new_tokens():
    c = workloads.decode_qwen3_8b("cuda", batch=64)
    _check(c.k_new, c.v_new, c.k_cache[0], c.v_cache[0], c.slot_mapping)


def test_prefill_padded_batch_with_negative_slots():
    """Padded (B, S_max) prefill step: -1 slots of the padding are skipped."""
    lens = workloads.uniform_lengths(8, 256, 4096, 3003)
    bs, nb = 16, 4096
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(7)).tolist()
    queries, off = [], 0
    for L in lens:
        n = -(-L // bs)
        queries.append(meta.Query(L, 0, meta.PREFILL, perm[off:off + n], bs))
        off += n
    md = meta.build(queries)
    slots = md["slot_mapping"].cuda()
    b, s = slots.shape
    g = torch.Generator(device="cuda").manual_seed(11)
    k = torch.randn((b, s, 8, 128), generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn((b, s, 8, 128), generator=g, device="cuda").to(torch.bfloat16)
    kc = torch.randn((nb, 8, bs, 128), generator=g, device="cuda").to(torch.bfloat16)
    vc = torch.randn((nb, 8, bs, 128), generator=g, device="cuda").to(torch.bfloat16)
    _check(k, v, kc, vc, slots)


def test_strided_kv_from_fused_projection():
    """k and v as views into one fused (T, 3, H, D) tensor (16-byte aligned rows)."""
    g = torch.Generator(device="cuda").manual_seed(3)
    t, hkv, d, bs, nb = 37, 4, 128, 16, 64
    fused = torch.randn((t, 3, hkv, d), generator=g, device="cuda").to(torch.bfloat16)
    k, v = fused[:, 1], fused[:, 2]
    slots = torch.randperm(nb * bs, generator=torch.Generator().manual_seed(5))[:t]
    slots[::5] = -1
    kc = torch.zeros((nb, hkv, bs, d), dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    _check(k.unsqueeze(0), v.unsqueeze(0), kc, vc, slots.view(1, t).cuda())


def test_misaligned_rows_take_narrow_copies():
    """head_dim 4 in fp32 (16-byte rows) and head_dim 6 in bf16 (12-byte rows)."""
    g = torch.Generator(device="cuda").manual_seed(9)
    for dtype, d in ((torch.float32, 4), (torch.bfloat16, 6)):
        k = torch.randn((1, 10, 2, d), generator=g, device="cuda").to(dtype)
        v = torch.randn((1, 10, 2, d), generator=g, device="cuda").to(dtype)
        kc = torch.zeros((8, 2, 4, d), dtype=dtype, device="cuda")
        vc = torch.zeros_like(kc)
        slots = torch.tensor([[0, 3, 5, -1, 31, 7, 8, 9, 10, -1]], device="cuda")
        _check(k, v, kc, vc, slots)


def test_out_of_range_slots_are_skipped():
    kc = torch.zeros((4, 2, 16, 128), dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    k = torch.ones((1, 3, 2, 128), dtype=torch.bfloat16, device="cuda")
    slots = torch.tensor([[64, 1000, 5]], device="cuda")
    ops.kv_write(k, k, kc, vc, slots)
    torch.cuda.synchronize()
    flat = kc.permute(0, 2, 1, 3).reshape(64, 2, 128)
    assert flat[5].eq(1).all() and flat.sum().item() == 2 * 128
