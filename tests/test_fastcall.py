"""The CPython fast-call module makes the same calls as the ctypes binding (CPU).

No kernel is launched: the calls compared are ones the library's argument
validation answers before touching the GPU.
"""
import ctypes

import pytest

from nano_inference_amd import _lib

KIND = {ctypes.c_void_p: "p", ctypes.c_int64: "l", ctypes.c_int32: "i", ctypes.c_float: "f",
        ctypes.c_size_t: "z"}


@pytest.fixture(scope="module")
def fast():
    mod = _lib.fast_module()
    assert mod is not None, "_nia_fast is not built (build_lib.build() compiles it)"
    assert _lib.calls() is mod
    return mod


def test_argument_kinds_follow_the_ctypes_signatures(fast):
    assert set(fast.kinds) == set(_lib.FAST_CALLS)
    for name in _lib.FAST_CALLS:
        res, args = _lib.SIGNATURES[name]
        assert res is ctypes.c_int32, name
        assert fast.kinds[name] == "".join(KIND[a] for a in args), name


def test_a_module_built_for_other_signatures_is_not_used(fast, monkeypatch):
    """A stale _nia_fast (argument kinds that no longer match SIGNATURES) must not be
    bound: its calls would pass the arguments in the wrong layout."""
    stale = dict(fast.kinds)
    stale["nia_paged_decode"] = stale["nia_paged_decode"][:-1]  # one argument fewer
    monkeypatch.setattr(fast, "kinds", stale)
    with pytest.warns(RuntimeWarning, match="does not match"):
        assert _lib.fast_module() is None
    monkeypatch.setattr(fast, "kinds", dict(fast.kinds, nia_prefill="p" * 25))
    with pytest.warns(RuntimeWarning):
        assert _lib.fast_module() is None


P = 16  # a pointer value validation rejects before any use


def early_return_cases():
    """(name, args) pairs whose status the library decides without a launch."""
    kv = [P, 0, 0, P, 0, 0, P, P, P, 4, 8, 128, 16, 10, 0, None]
    dec = [P, 0, 0, P, 0, 0, P, P, P, 4, 4, P, 2, 8, 4, 128, 16, 10, 0.1, None, 0, 0, None]
    dec8 = [P, 0, 0, P, 0, 0, P, P, P, P, P, 4, 4, P, 2, 8, 4, 128, 16, 10, 0.1, None, 0, None]
    pf = [P, 8, 8, P, 8, 8, P, 8, 8, P, 8, 8, P, P, P, P, 1, 4, 2, 2, 128, 0.1, 1, 0, None]
    pp = [P, 8, 8, P, 8, 8, P, P, P, 4, 4, P, P, P, 1, 4, 2, 2, 128, 16, 10, 0.1, 2, 0, None]
    qk = [P, 1024, 128, P, 512, 128, P, 512, 128, None, None, 1e-6, P, 8, 1, P, 0, 0, None,
          None, None, 8, 8, 4, 128, 16, 10, 0, None]
    qk8 = qk[:20] + [P, P] + qk[20:]

    def with_(args, **at):
        a = list(args)
        for i, v in at.items():
            a[int(i[1:])] = v
        return a

    return [
        ("nia_kv_write", with_(kv, a9=-1)),                    # negative token count
        ("nia_kv_write", with_(kv, a9=0)),                     # nothing to do
        ("nia_kv_write", with_(kv, a14=7)),                    # unknown dtype
        ("nia_kv_write_fp8", [P, 0, 0, P, 0, 0, P, P, P, P, P, -1, 8, 128, 16, 10, 0, None]),
        ("nia_kv_write_fp8", [P, 0, 0, P, 0, 0, P, P, P, P, P, 0, 8, 128, 16, 10, 0, None]),
        ("nia_paged_decode", with_(dec, a13=6)),               # heads not divisible
        ("nia_paged_decode", with_(dec, a15=72)),              # head_dim
        ("nia_paged_decode", with_(dec, a12=0)),               # empty batch
        ("nia_paged_decode", with_(dec, a12=-1)),
        ("nia_paged_decode", [P, 128, 128, P, 1024, 128, P, P, P, 64, 64, P, 2, 8, 4, 128, 16,
                              100, 0.1, None, 0, 0, None]),    # workspace too small
        ("nia_paged_decode_fp8", with_(dec8, a15=6)),
        ("nia_paged_decode_fp8", with_(dec8, a17=72)),
        ("nia_prefill", with_(pf, a23=7)),                     # unknown dtype
        ("nia_prefill", with_(pf, a4=6, a23=1)),               # fp32 rows break 16 B loads
        ("nia_prefill", with_(pf, a22=5)),                     # causal mode
        ("nia_prefill", with_(pf, a21=0.0)),                   # scale
        ("nia_prefill_paged", with_(pp, a19=12)),              # block size
        ("nia_prefill_paged", with_(pp, a14=-1)),
        ("nia_qk_norm_rope_kv_write", with_(qk, a21=0)),
        ("nia_qk_norm_rope_kv_write", with_(qk, a21=-1)),
        ("nia_qk_norm_rope_kv_write", with_(qk, a14=2)),
        ("nia_qk_norm_rope_kv_write", with_(qk, a24=64)),
        ("nia_qk_norm_rope_kv_write", with_(qk, a18=P)),       # k_cache without v_cache
        ("nia_qk_norm_rope_kv_write_fp8", with_(qk8, a23=-1)),
        ("nia_qk_norm_rope_kv_write_fp8", with_(qk8, a26=64)),
    ]


def test_same_status_as_ctypes_on_early_returns(fast):
    lib = _lib.load()
    statuses = set()
    for name, args in early_return_cases():
        assert len(args) == len(fast.kinds[name]), name
        want = getattr(lib, name)(*args)
        got = getattr(fast, name)(*args)
        assert got == want, (name, args, got, want)
        statuses.add(got)
    # the cases reach several distinct answers, not one default
    assert {_lib.OK, _lib.ERR_INVALID_ARGUMENT, _lib.ERR_UNSUPPORTED} <= statuses


def test_argument_errors_raise_instead_of_truncating(fast):
    _, args = early_return_cases()[0]
    with pytest.raises(TypeError):
        fast.nia_kv_write(*args[:-1])
    with pytest.raises(OverflowError):
        fast.nia_kv_write(*args[:9], 1 << 40, *args[10:])      # an int32 argument
    with pytest.raises(TypeError):
        fast.nia_kv_write("x", *args[1:])                      # a pointer that is no int
    with pytest.raises(KeyError):
        fast.bind("nia_abi_version", 1)
