"""Pins oracle.qk_rope (QK-RMSNorm, RoPE, mRoPE) before it checks the fused kernel.

- The reference's own unit tests for these modules, restated against the oracle:
  tests/unit/test_norm.py (shape, RMS ~ 1, the x = 1..4 formula),
  tests/unit/test_rotary.py (norm preserved, position 0 is the identity),
  tests/unit/test_mrope.py (text tokens == 1-D RoPE, image tokens differ, bad
  section rejected).
- Closed forms: a unit vector e_i at position p rotates to cos(p w_i) e_i +
  sin(p w_i) e_{i+D/2}, and e_{i+D/2} to -sin e_i + cos e_{i+D/2}; the x = 1..4
  RMSNorm value; for mRoPE, frequency i takes its angle from axis t (i < n_t),
  h (i < n_t + n_h) or w.
- Invariant: <R(m) q, R(n) k> depends only on m - n (float64).
- Planted mistakes (a flipped sign, adjacent-pair rotation, swapped mRoPE axes,
  a dropped eps) fail at least one of the checks above.
"""
import math

import pytest
import torch

from oracle import qk_rope as O

D = 128
BASE = 1e6


def unit_rotation_ok(rope_fn, freqs, pos, atol=1e-12):
    """Closed form of the rotation on every unit vector (float64)."""
    eye = torch.eye(D, dtype=torch.float64).view(1, D, 1, D)  # B=1, S=D tokens, H=1
    p = torch.full((1, D), float(pos), dtype=torch.float64)
    out, _ = rope_fn(eye, eye, p, freqs)
    out = out[0, :, 0, :]
    h = D // 2
    for i in range(D):
        j = i % h
        ang = pos * float(freqs[j])
        exp = torch.zeros(D, dtype=torch.float64)
        if i < h:
            exp[i], exp[i + h] = math.cos(ang), math.sin(ang)
        else:
            exp[j], exp[i] = -math.sin(ang), math.cos(ang)
        if not torch.allclose(out[i], exp, atol=atol, rtol=0):
            return False
    return True


def test_rms_norm_kats():
    w = torch.ones(16)
    x = torch.randn(2, 4, 16)
    assert O.rms_norm(x, w, 1e-6).shape == x.shape
    x = torch.randn(1, 1, 64) * 10.0
    out = O.rms_norm(x, torch.ones(64), 1e-6)
    rms = out.pow(2).mean(-1).sqrt()
    torch.testing.assert_close(rms, torch.ones_like(rms), atol=1e-3, rtol=1e-3)
    x = torch.arange(1.0, 5.0)
    y = O.rms_norm(x, torch.ones(4), 1e-6)
    exp = torch.tensor([1.0, 2.0, 3.0, 4.0], dtype=torch.float64) / math.sqrt(7.5 + 1e-6)
    assert torch.allclose(y.double(), exp, atol=1e-6)


def test_rms_norm_weight_and_cast_points():
    x = torch.randn(3, 5, D).to(torch.bfloat16)
    w = (torch.randn(D) * 0.5 + 1).to(torch.bfloat16)
    y = O.rms_norm(x, w, 1e-6)
    assert y.dtype == torch.bfloat16
    # cast back before the weight: y == bf16(bf16(x * r) * w), computed independently
    r = 1.0 / torch.sqrt(x.double().pow(2).mean(-1, keepdim=True) + 1e-6)
    xn = (x.double() * r).float().to(torch.bfloat16)
    exp = (xn.float() * w.float()).to(torch.bfloat16)
    assert (y.view(torch.int16) != exp.view(torch.int16)).float().mean() < 1e-3
    assert (y.float() - exp.float()).abs().max() <= 2 ** -6 * exp.float().abs().max()


def test_rope_kats():
    freqs = O.inv_freq(16, 1e4)
    q, k = torch.randn(1, 4, 2, 16), torch.randn(1, 4, 2, 16)
    qo, ko = O.rope(q, k, torch.tensor([[0, 1, 2, 3]]), freqs)
    assert qo.shape == q.shape and ko.shape == k.shape
    freqs = O.inv_freq(8, 1e4)
    q, k = torch.randn(1, 1, 1, 8), torch.randn(1, 1, 1, 8)
    qo, ko = O.rope(q, k, torch.tensor([[5]]), freqs)
    torch.testing.assert_close(q.norm(), qo.norm())
    torch.testing.assert_close(k.norm(), ko.norm())
    q, k = torch.randn(1, 1, 2, 8), torch.randn(1, 1, 2, 8)
    qo, ko = O.rope(q, k, torch.zeros((1, 1)), freqs)
    torch.testing.assert_close(qo, q)
    torch.testing.assert_close(ko, k)


def test_inv_freq_closed_form():
    f = O.inv_freq(D, BASE).double()
    exp = torch.tensor([BASE ** (-2 * i / D) for i in range(D // 2)], dtype=torch.float64)
    assert torch.allclose(f, exp, rtol=1e-6, atol=0)


@pytest.mark.parametrize("pos", [0, 1, 7, 1000, 40000])
def test_rope_closed_form_on_unit_vectors(pos):
    assert unit_rotation_ok(O.rope, O.inv_freq(D, BASE).double(), pos)


def test_rope_relative_position_invariance():
    g = torch.Generator().manual_seed(0)
    f = O.inv_freq(D, BASE).double()
    q = torch.randn(1, 1, 1, D, generator=g, dtype=torch.float64)
    k = torch.randn(1, 1, 1, D, generator=g, dtype=torch.float64)

    def dot(m, n):
        qm, _ = O.rope(q, q, torch.tensor([[m]]), f)
        kn, _ = O.rope(k, k, torch.tensor([[n]]), f)
        return float((qm * kn).sum())

    for m, n, t in [(5, 2, 100), (300, 17, 4096), (9, 9, 12345)]:
        assert dot(m, n) == pytest.approx(dot(m + t, n + t), rel=1e-9, abs=1e-9)


def test_mrope_kats():
    f = O.inv_freq(D, BASE)
    sec = (16, 24, 24)
    B, S, H = 2, 8, 4
    q, k = torch.randn(B, S, H, D), torch.randn(B, S, H, D)
    p1 = torch.arange(S).unsqueeze(0).expand(B, -1)
    q1, k1 = O.rope(q.clone(), k.clone(), p1, f)
    qm, km = O.mrope(q.clone(), k.clone(), p1.unsqueeze(0).expand(3, -1, -1), f, sec)
    assert torch.allclose(q1, qm, atol=1e-5) and torch.allclose(k1, km, atol=1e-5)
    q, k = torch.randn(1, 4, 4, D), torch.randn(1, 4, 4, D)
    p3 = torch.tensor([[[0, 0, 0, 0]], [[0, 0, 1, 1]], [[0, 1, 0, 1]]])
    q1, _ = O.rope(q.clone(), k.clone(), p3[0], f)
    qm, _ = O.mrope(q.clone(), k.clone(), p3, f, sec)
    assert not torch.allclose(q1, qm, atol=1e-5)
    with pytest.raises(ValueError):
        O.mrope(q, k, p3, f, (10, 10, 10))


def test_mrope_axis_selection_closed_form():
    f = O.inv_freq(D, BASE).double()
    sec = (16, 24, 24)
    pos_axes = (3, 50, 700)
    eye = torch.eye(D, dtype=torch.float64).view(1, D, 1, D)
    p3 = torch.tensor(pos_axes, dtype=torch.float64).view(3, 1, 1).expand(3, 1, D)
    out, _ = O.mrope(eye, eye, p3, f, sec)
    out = out[0, :, 0, :]
    for i in range(D // 2):
        axis = 0 if i < 16 else (1 if i < 40 else 2)
        ang = pos_axes[axis] * float(f[i])
        assert out[i, i] == pytest.approx(math.cos(ang), abs=1e-12)
        assert out[i, i + 64] == pytest.approx(math.sin(ang), abs=1e-12)


def test_planted_mistakes_fail():
    f = O.inv_freq(D, BASE).double()

    def rope_sign_flip(q, k, p, fr):
        freqs = p.double().unsqueeze(-1) * fr
        emb = torch.cat((freqs, freqs), -1)
        c, s = emb.cos().unsqueeze(2), emb.sin().unsqueeze(2)
        rh = lambda x: torch.cat((x[..., D // 2:], -x[..., :D // 2]), -1)  # wrong sign
        return q * c + rh(q) * s, k * c + rh(k) * s

    def rope_adjacent_pairs(q, k, p, fr):
        freqs = p.double().unsqueeze(-1) * fr
        emb = freqs.repeat_interleave(2, -1)  # interleaved layout instead of halves
        c, s = emb.cos().unsqueeze(2), emb.sin().unsqueeze(2)

        def rh(x):
            x2 = x.view(*x.shape[:-1], D // 2, 2)
            return torch.stack((-x2[..., 1], x2[..., 0]), -1).view_as(x)
        return q * c + rh(q) * s, k * c + rh(k) * s

    assert unit_rotation_ok(O.rope, f, 7)
    assert not unit_rotation_ok(rope_sign_flip, f, 7)
    assert not unit_rotation_ok(rope_adjacent_pairs, f, 7)
    # swapped h and w sections must break the axis closed form
    eye = torch.eye(D, dtype=torch.float64).view(1, D, 1, D)
    p3 = torch.tensor((3, 50, 700), dtype=torch.float64).view(3, 1, 1).expand(3, 1, D)
    good, _ = O.mrope(eye, eye, p3, f, (16, 24, 24))
    swapped, _ = O.mrope(eye, eye, p3[[0, 2, 1]], f, (16, 24, 24))
    assert not torch.allclose(good, swapped)
    # RMSNorm without eps differs from the x = 1..4 closed form at a tiny scale
    x = torch.arange(1.0, 5.0, dtype=torch.float64) * 1e-4
    good = O.rms_norm(x, torch.ones(4, dtype=torch.float64), 1e-6)
    no_eps = x / x.pow(2).mean().sqrt()
    exp = x / math.sqrt(7.5e-8 + 1e-6)
    assert torch.allclose(good.double(), exp, rtol=1e-6)
    assert not torch.allclose(no_eps, exp, rtol=1e-3)
