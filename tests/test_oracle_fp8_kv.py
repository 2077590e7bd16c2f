"""Pins the fp8 KV-cache oracle (oracle/fp8_kv.py) on the CPU.

- torch's float8_e4m3fn conversion (the library routine the oracle uses) against
  the format's definition: every one of the 256 codes decodes to the value the
  e4m3 formula gives, and every midpoint between neighbouring values rounds to the
  even code (round to nearest even), the largest finite value being 448.
- Row quantisation: the largest magnitude of a row maps to +-448 exactly; rows of
  exactly representable values (times a power of two) round-trip exactly; the
  error of every element is at most half a unit in the last place of its code
  times the scale (relative 2^-4 of the element, or 2^-10 of the row maximum for
  subnormal codes); zero rows give scale 0 and zero codes.
- A planted mistake (scale = max / 256, or truncation instead of rounding) breaks
  one of these checks.
- The fp8 write loop puts each quantised row at its slot and skips -1 slots.
"""
import math

import numpy as np
import pytest
import torch

from oracle import fp8_kv as F


def test_codes_decode_to_the_format_definition():
    got = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().tolist()
    for c in range(256):
        want = F.e4m3_value(c)
        if math.isnan(want):
            assert math.isnan(got[c]), c
        else:
            assert got[c] == want, (c, got[c], want)
    assert max(v for v in got if not math.isnan(v)) == 448.0


def test_midpoints_round_to_even():
    vals = sorted({F.e4m3_value(c) for c in range(128) if not math.isnan(F.e4m3_value(c))})
    codes = {F.e4m3_value(c): c for c in range(128)}
    for a, b in zip(vals[:-1], vals[1:]):
        mid = (a + b) / 2
        got = torch.tensor([mid], dtype=torch.float32).to(torch.float8_e4m3fn).view(
            torch.uint8).item()
        even = codes[a] if codes[a] % 2 == 0 else codes[b]
        assert got == even, (a, b, got, even)


def test_row_max_maps_to_448_and_error_bound():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(200, 128, generator=g) * torch.logspace(-3, 3, 200).unsqueeze(1)
    q, s = F.quantize_rows(x)
    deq = F.dequantize_rows(q, s)
    amax = x.abs().amax(-1)
    arg = x.abs().argmax(-1)
    codes = q.gather(1, arg.unsqueeze(1)).squeeze(1)
    assert torch.all((codes & 0x7F) == 0x7E), "row max must be the 448 code"
    err = (deq - x).abs()
    # half an ulp of each code: 2^-4 relative for normal codes, 2^-10 * scale below 2^-6
    rel = torch.maximum(x.abs() * 2.0 ** -4, (s * 2.0 ** -10).unsqueeze(1))
    assert torch.all(err <= rel * (1 + 1e-6)), float((err / rel).max())
    assert torch.allclose(s, amax / 448.0)


def test_representable_rows_round_trip_exactly():
    vals = [F.e4m3_value(c) for c in range(0x7F) if not math.isnan(F.e4m3_value(c))]
    row = torch.tensor(vals[:127] + [448.0], dtype=torch.float32)
    for p in (-20, 0, 7):
        x = row * 2.0 ** p
        q, s = F.quantize_rows(x.unsqueeze(0))
        assert s.item() == 2.0 ** p
        assert torch.equal(F.dequantize_rows(q, s)[0], x)


def test_zero_rows():
    q, s = F.quantize_rows(torch.zeros(3, 128))
    assert torch.all(s == 0) and torch.all(q == 0)
    assert torch.all(F.dequantize_rows(q, s) == 0)


def test_planted_mistakes_fail():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(64, 128, generator=g)
    # wrong scale constant: the row max no longer lands on 448
    s_bad = x.abs().amax(-1) / 256.0
    q_bad = (x / s_bad.unsqueeze(1)).to(torch.float8_e4m3fn).view(torch.uint8)
    arg = x.abs().argmax(-1)
    assert not torch.all((q_bad.gather(1, arg.unsqueeze(1)) & 0x7F) == 0x7E)
    # truncation instead of rounding breaks the half-ulp bound somewhere
    s = x.abs().amax(-1) / 448.0
    y = x / s.unsqueeze(1)
    e = torch.floor(torch.log2(y.abs().clamp(min=2.0 ** -6)))
    step = 2.0 ** (e - 3)
    trunc = torch.sign(y) * torch.floor(y.abs() / step) * step
    err = (trunc * s.unsqueeze(1) - x).abs()
    assert torch.any(err > x.abs() * 2.0 ** -4 * 1.01)


def test_write_loop_places_rows_and_skips_padding():
    g = torch.Generator().manual_seed(2)
    k = torch.randn(2, 5, 3, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(2, 5, 3, 128, generator=g).to(torch.bfloat16)
    kc = torch.zeros(8, 3, 4, 128, dtype=torch.uint8)
    vc = torch.zeros_like(kc)
    ks = torch.zeros(8, 3, 4)
    vs = torch.zeros_like(ks)
    slots = torch.tensor([[0, 1, 2, 7, -1], [12, 13, -1, -1, 30]])
    F.kv_write_loop_fp8(k, v, kc, vc, ks, vs, slots)
    for b in range(2):
        for s in range(5):
            sl = int(slots[b, s])
            if sl < 0:
                continue
            qk, sk = F.quantize_rows(k[b, s])
            assert torch.equal(kc[sl // 4, :, sl % 4], qk) and torch.equal(ks[sl // 4, :, sl % 4], sk)
    written = {int(s) for s in slots.flatten() if s >= 0}
    for sl in range(32):
        if sl not in written:
            assert torch.all(kc[sl // 4, :, sl % 4] == 0) and torch.all(vs[sl // 4, :, sl % 4] == 0)
    np.testing.assert_array_equal(vc[7 // 4, :, 7 % 4].numpy(), F.quantize_rows(v[0, 3])[0].numpy())
