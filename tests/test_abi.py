"""The C-ABI library loads and exports every symbol include/nia_attn.h declares (CPU).

No kernel is launched: only entry points that return before touching the GPU
(argument validation, sizes, strings) are called.
"""
import ctypes
import os
import re

from nano_inference_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "nia_attn.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nia_\w+)\s*\(", text)))


def test_every_declared_symbol_is_exported_and_bound():
    lib = _lib.load()
    names = header_functions()
    assert len(names) >= 7
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


def test_version_and_error_strings():
    lib = _lib.load()
    assert lib.nia_abi_version() == _lib.ABI_VERSION
    for code in range(7):
        assert lib.nia_error_string(code)
    assert lib.nia_error_string(0) == b"ok"
    assert lib.nia_error_string(99) == b"unknown status"


def test_validation_returns_codes_without_launching():
    lib = _lib.load()
    # negative token count
    assert lib.nia_kv_write(None, 0, 0, None, 0, 0, None, None, None, -1, 8, 128, 16, 10,
                            0, None) == _lib.ERR_INVALID_ARGUMENT
    # zero tokens: nothing to do
    assert lib.nia_kv_write(None, 0, 0, None, 0, 0, None, None, None, 0, 8, 128, 16, 10,
                            0, None) == _lib.OK
    # unsupported dtype
    assert lib.nia_kv_write(None, 0, 0, None, 0, 0, None, None, None, 1, 8, 128, 16, 10,
                            7, None) == _lib.ERR_UNSUPPORTED
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    # decode: heads not divisible
    assert lib.nia_paged_decode(p, 0, 0, p, 0, 0, p, p, p, 4, 4, p, 2, 6, 4, 128, 16, 10, 0.1,
                                None, 0, 0, None) == _lib.ERR_INVALID_ARGUMENT
    # decode: unsupported head_dim, also at a block size the split kernels do not take
    assert lib.nia_paged_decode(p, 0, 0, p, 0, 0, p, p, p, 4, 4, p, 2, 8, 4, 72, 16, 10, 0.1,
                                None, 0, 0, None) == _lib.ERR_UNSUPPORTED
    assert lib.nia_paged_decode(p, 0, 0, p, 0, 0, p, p, p, 4, 4, p, 2, 8, 4, 72, 12, 10, 0.1,
                                None, 0, 0, None) == _lib.ERR_UNSUPPORTED
    # bf16 block size 2 takes the any-size kernel and 12 the split kernels: both refuse a q
    # that is not 8-byte aligned
    odd = ctypes.c_void_p(18)
    for bs in (2, 12):
        assert lib.nia_paged_decode(p, 0, 0, odd, 0, 0, p, p, p, 4, 4, p, 2, 8, 4, 128, bs, 10,
                                    0.1, p, 1 << 30, 0, None) == _lib.ERR_MISALIGNED
    # a group of 32 is a supported shape: validation gets as far as the workspace alignment
    assert lib.nia_paged_decode(p, 0, 0, p, 0, 0, p, p, p, 4, 4, p, 2, 32, 1, 128, 16, 10, 0.1,
                                p, 1 << 30, 0, None) == _lib.ERR_MISALIGNED
    # decode: 2^16 sequences over a table 2^24 keys wide: 2^35 units of 32 keys, beyond the
    # split kernel's int prefix sums
    ws = ctypes.c_void_p(4096)
    assert lib.nia_paged_decode(p, 0, 0, p, 0, 0, p, p, p, 1 << 20, 1 << 20, p, 1 << 16, 32, 8,
                                128, 16, 10, 0.1, ws, 1 << 40, 0, None) == _lib.ERR_UNSUPPORTED
    # decode: workspace too small for 2 partitions
    assert lib.nia_paged_decode(p, 128, 128, p, 1024, 128, p, p, p, 64, 64, p, 2, 8, 4, 128, 16,
                                100, 0.1, None, 0, 0, None) == _lib.ERR_WORKSPACE
    # prefill: unknown dtype; fp32 rows whose strides break 16-byte loads
    assert lib.nia_prefill(p, 8, 8, p, 8, 8, p, 8, 8, p, 8, 8, p, p, p, p, 1, 4, 2, 2, 128, 0.1,
                           1, 7, None) == _lib.ERR_UNSUPPORTED
    assert lib.nia_prefill(p, 8, 8, p, 6, 8, p, 8, 8, p, 8, 8, p, p, p, p, 1, 4, 2, 2, 128, 0.1,
                           1, 1, None) == _lib.ERR_MISALIGNED
    # prefill: bad causal mode, non-positive scale
    assert lib.nia_prefill(p, 8, 8, p, 8, 8, p, 8, 8, p, 8, 8, p, p, p, p, 1, 4, 2, 2, 128, 0.1,
                           5, 0, None) == _lib.ERR_INVALID_ARGUMENT
    assert lib.nia_prefill(p, 8, 8, p, 8, 8, p, 8, 8, p, 8, 8, p, p, p, p, 1, 4, 2, 2, 128, 0.0,
                           1, 0, None) == _lib.ERR_INVALID_ARGUMENT
    # paged prefill: a bf16 block size that is not a power of two takes the MFMA kernels
    # (their checks see the unaligned q); an unsupported head_dim is refused first
    assert lib.nia_prefill_paged(p, 8, 8, ctypes.c_void_p(18), 8, 8, p, p, p, 4, 4, p, p, p, 1,
                                 4, 2, 2, 128, 12, 10, 0.1, 2, 0, None) == _lib.ERR_MISALIGNED
    assert lib.nia_prefill_paged(p, 8, 8, p, 8, 8, p, p, p, 4, 4, p, p, p, 1, 4, 2, 2, 72, 12,
                                 10, 0.1, 2, 0, None) == _lib.ERR_UNSUPPORTED


def test_noalloc_decode_refuses_sizes_beyond_its_scratch_without_launching():
    lib = _lib.load()
    p = ctypes.c_void_p(16)  # never dereferenced: the size check comes first
    # fp32 partitions: 4096 sequences x 64 heads x 256 partitions, far beyond the array
    need = lib.nia_paged_decode_workspace_size(4096, 64, 8, 8192, 16, 128, 1)
    assert need > _lib.DECODE_SCRATCH_BYTES
    assert lib.nia_paged_decode_noalloc(p, 0, 0, p, 0, 0, p, p, p, 8192, 8192, p, 4096, 64, 8,
                                        128, 16, 10, 0.1, 1, None) == _lib.ERR_SCRATCH_LIMIT
    assert lib.nia_paged_decode_noalloc(p, 0, 0, p, 0, 0, p, p, p, 4, 4, p, 0, 8, 4, 128, 16,
                                        10, 0.1, 0, None) == _lib.OK  # empty batch
    assert lib.nia_paged_decode_noalloc(p, 0, 0, p, 0, 0, p, p, p, 4, 4, p, -1, 8, 4, 128, 16,
                                        10, 0.1, 0, None) == _lib.ERR_INVALID_ARGUMENT


def test_workspace_size():
    lib = _lib.load()
    hdr = 256
    # bf16 (and fp8): the unit prefix (batch + 1 ints, rounded to 256 B), the merge's range
    # records (2 ints per sequence and KV head, rounded to 256 B), then (m, l) and the
    # partial output of 8 G rows per workgroup for a grid of at most 512
    pfx = -(-(64 + 1) * 4 // 256) * 256
    rec = -(-(64 * 8 * 2 * 4) // 256) * 256
    assert lib.nia_paged_decode_workspace_size(64, 32, 8, 512, 16, 128, 0) == \
        hdr + pfx + rec + 512 * 8 * 4 * 130 * 4
    assert lib.nia_paged_decode_workspace_size(64, 32, 8, 32, 16, 80, 0) == \
        hdr + pfx + rec + 512 * 8 * 4 * 82 * 4
    rec3 = -(-(5 * 3 * 2 * 4) // 256) * 256
    assert lib.nia_paged_decode_workspace_size(5, 6, 3, 32, 16, 128, 0) == \
        hdr + 256 + rec3 + 512 * 8 * 2 * 130 * 4
    # fp32 at head_dim 128 / block 16: partitions of 32 blocks per (sequence, head)
    assert lib.nia_paged_decode_workspace_size(64, 32, 8, 32, 16, 128, 1) == \
        hdr + 64 * 32 * 130 * 4
    assert lib.nia_paged_decode_workspace_size(64, 32, 8, 512, 16, 128, 1) == \
        hdr + 64 * 32 * 16 * 130 * 4
    # fp32 other shapes run without partials
    assert lib.nia_paged_decode_workspace_size(64, 32, 8, 512, 32, 128, 1) == hdr
    # bf16 block sizes the split kernels do not take (not multiples of 4) run the any-size
    # kernel, without partials either; multiples of 4 take the split kernels' workspace
    for bs in (1, 2, 3, 5, 6, 10, 22):
        assert lib.nia_paged_decode_workspace_size(64, 32, 8, 512, bs, 128, 0) == hdr
    for bs in (12, 24, 48, 100):
        assert lib.nia_paged_decode_workspace_size(64, 32, 8, 512, bs, 128, 0) == \
            hdr + pfx + rec + 512 * 8 * 4 * 130 * 4
    assert lib.nia_paged_decode_workspace_size(64, 32, 3, 512, 16, 128, 0) == 0  # 32 % 3


def test_qk_norm_rope_validation_without_launching():
    lib = _lib.load()
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails or returns first
    args = dict(q=p, qt=1024, qh=128, k=p, kt=512, kh=128, v=p, vt=512, vh=128, qw=None, kw=None,
                eps=1e-6, pos=p, pax=8, axes=1, inv=p, s0=0, s1=0, kc=None, vc=None, sl=None,
                n=8, h=8, hkv=4, d=128, bs=16, nb=10, dt=0, st=None)

    def call(**kw):
        a = dict(args, **kw)
        return lib.nia_qk_norm_rope_kv_write(*a.values())

    assert call(n=0) == _lib.OK
    assert call(n=-1) == _lib.ERR_INVALID_ARGUMENT
    assert call(axes=2) == _lib.ERR_INVALID_ARGUMENT
    assert call(axes=3, s0=40, s1=40) == _lib.ERR_INVALID_ARGUMENT  # sections exceed D/2
    assert call(qw=p, kw=p, eps=-1.0) == _lib.ERR_INVALID_ARGUMENT
    assert call(kc=p) == _lib.ERR_INVALID_ARGUMENT  # a cache write needs v_cache and slots
    assert call(d=64) == _lib.ERR_UNSUPPORTED
    assert call(dt=7) == _lib.ERR_UNSUPPORTED


def test_step_metadata_validation_without_launching():
    lib = _lib.load()
    p = ctypes.c_void_p(16)  # never dereferenced
    args = [p, 10, 4, 0, 2, 5, 9, 3, 16, p, p, p, p, p, p, p, None, None]
    assert lib.nia_step_metadata(*args[:4], 0, *args[5:]) == _lib.OK          # empty batch
    assert lib.nia_step_metadata(*args[:4], -1, *args[5:]) == _lib.ERR_INVALID_ARGUMENT
    assert lib.nia_step_metadata(*args[:8], 0, *args[9:]) == _lib.ERR_INVALID_ARGUMENT  # BS 0
    assert lib.nia_step_metadata(None, *args[1:]) == _lib.ERR_INVALID_ARGUMENT
    assert lib.nia_step_metadata(*args[:4], 70000, *args[5:]) == _lib.ERR_UNSUPPORTED
