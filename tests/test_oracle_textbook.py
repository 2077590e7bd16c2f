"""Pins of oracle.textbook: brute force, closed forms and planted mistakes (CPU)."""
import math

import numpy as np
import pytest

from oracle import textbook as tb


def rnd(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


@pytest.mark.parametrize("n,m,d", [(1, 1, 4), (3, 5, 8), (7, 7, 6), (4, 9, 16)])
@pytest.mark.parametrize("mode", ["none", "top_left", "bottom_right"])
def test_attend_matches_bruteforce(n, m, d, mode):
    q, k, v = rnd((n, d), 1), rnd((m, d), 2), rnd((m, d), 3)
    bounds = tb.causal_bounds(n, m, mode)
    got = tb.attend(q, k, v, 1 / math.sqrt(d), bounds)
    ref = np.array(tb.attend_bruteforce(q.tolist(), k.tolist(), v.tolist(), 1 / math.sqrt(d),
                                        bounds.tolist()))
    np.testing.assert_allclose(got, ref, atol=1e-12)


def test_causal_bounds_definitions():
    # top-left on a square matrix is the reference's triu(diagonal=1) mask
    tri = np.triu(np.ones((6, 6), dtype=bool), k=1)
    assert (tb.causal_bounds(6, 6, "top_left") == (~tri).sum(1)).all()
    # bottom-right: the last query row sees every key; square case equals top-left
    assert tb.causal_bounds(3, 10, "bottom_right").tolist() == [8, 9, 10]
    assert (tb.causal_bounds(5, 5, "bottom_right") == tb.causal_bounds(5, 5, "top_left")).all()
    # top-left rows past the key count see all keys (padded prefill rows)
    assert tb.causal_bounds(5, 3, "top_left").tolist() == [1, 2, 3, 3, 3]
    # more queries than keys bottom-right: leading rows see nothing
    assert tb.causal_bounds(4, 2, "bottom_right").tolist() == [0, 0, 1, 2]


def test_closed_forms():
    d = 8
    q, k, v = rnd((5, d), 4), rnd((10, d), 5), rnd((10, d), 6)
    # one key: output is that key's value, whatever q
    np.testing.assert_allclose(tb.attend(q, k[:1], v[:1], 0.3), np.repeat(v[:1], 5, 0), atol=1e-15)
    # identical keys: uniform weights, output is the mean of V
    kk = np.repeat(k[:1], 10, 0)
    np.testing.assert_allclose(tb.attend(q, kk, v, 0.3), np.repeat(v.mean(0, keepdims=True), 5, 0),
                               atol=1e-14)
    # constant V: output is that constant
    vc = np.full((10, d), 1.75)
    np.testing.assert_allclose(tb.attend(q, k, vc, 0.3), vc[:5], atol=1e-14)
    # one dominant key: output is (numerically) its value
    kd = k.copy()
    kd[4] = 1e3 * q[0]
    np.testing.assert_allclose(tb.attend(q[:1], kd, v, 1.0)[0], v[4], atol=1e-12)
    # zero visible keys: zeros
    assert (tb.attend(q, k, v, 0.3, np.zeros(5, int)) == 0).all()


def _planted_attend_no_scale(q, k, v, scale, bounds=None):
    return tb.attend(q, k, v, 1.0, bounds)


def _planted_attend_off_by_one(q, k, v, scale, bounds=None):
    return tb.attend(q, k, v, scale, None if bounds is None else np.maximum(bounds - 1, 0))


@pytest.mark.parametrize("bad", [_planted_attend_no_scale, _planted_attend_off_by_one])
def test_bruteforce_catches_planted_mistakes(bad):
    n, m, d = 6, 6, 8
    q, k, v = rnd((n, d), 7), rnd((m, d), 8), rnd((m, d), 9)
    bounds = tb.causal_bounds(n, m, "top_left")
    ref = np.array(tb.attend_bruteforce(q.tolist(), k.tolist(), v.tolist(), 1 / math.sqrt(d),
                                        bounds.tolist()))
    assert not np.allclose(bad(q, k, v, 1 / math.sqrt(d), bounds), ref, atol=1e-6)


def _cache_case(seed, lens, h=8, hkv=2, d=16, bs=4, nb=40):
    rng = np.random.default_rng(seed)
    kc, vc = rng.standard_normal((nb, hkv, bs, d)), rng.standard_normal((nb, hkv, bs, d))
    perm = rng.permutation(nb)
    mb = max(-(-L // bs) for L in lens)
    bt = np.zeros((len(lens), mb), dtype=np.int64)
    off = 0
    for i, L in enumerate(lens):
        n = -(-L // bs)
        bt[i, :n] = perm[off:off + n]
        off += n
    q = rng.standard_normal((len(lens), h, d))
    return q, kc, vc, bt, np.array(lens)


def test_paged_decode_gqa_equals_mha_and_catches_wrong_head_map():
    q, kc, vc, bt, lens = _cache_case(11, [5, 13, 1])
    g = q.shape[1] // kc.shape[1]
    out = tb.paged_decode(q, kc, vc, bt, lens, 0.25)
    mha = tb.paged_decode(q, np.repeat(kc, g, 1), np.repeat(vc, g, 1), bt, lens, 0.25)
    np.testing.assert_allclose(out, mha, atol=1e-14)
    # planted mistake: head h reading KV head h % H_kv instead of h // G
    wrong = tb.paged_decode(q, np.tile(kc, (1, g, 1, 1)), np.tile(vc, (1, g, 1, 1)), bt, lens, 0.25)
    assert not np.allclose(out, wrong, atol=1e-6)


def test_paged_decode_block_permutation_invariance():
    q, kc, vc, bt, lens = _cache_case(12, [7, 16, 17])
    out = tb.paged_decode(q, kc, vc, bt, lens, 0.25)
    perm = np.random.default_rng(3).permutation(kc.shape[0])
    k2, v2 = np.empty_like(kc), np.empty_like(vc)
    k2[perm], v2[perm] = kc, vc
    np.testing.assert_allclose(tb.paged_decode(q, k2, v2, perm[bt], lens, 0.25), out, atol=1e-14)


def test_chunk_rows_equal_full_causal_rows():
    rng = np.random.default_rng(5)
    total, p, h, d = 40, 25, 2, 8
    q, k, v = (rng.standard_normal((total, h, d)) for _ in range(3))
    full = tb.varlen(q, k, v, [0], [total], [0], [total], 0.3, "top_left")[0][1]
    chunk = tb.varlen(q, k, v, [p], [total - p], [0], [total], 0.3, "bottom_right")[0][1]
    np.testing.assert_allclose(chunk, full[p:], atol=1e-14)
