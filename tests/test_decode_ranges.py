"""The unit ranges of the split decode kernel, as its fp64 arithmetic forms them.

Virtual wave v of V owns units [start(v), start(v + 1)) with start(v) = floor(total * W(v) /
W(V)), W(v) summing per-wave weights (WF for the first `first` waves, WS for the rest).  The
kernel evaluates the quotient in fp64 and the combine kernel inverts it (the range holding
a unit) the same way; both are exact only while the products stay below 2^53 and a
non-integer quotient lies further from an integer than the rounding error.  The host
refuses batches of more than 2^36 units, so these checks run up to that size: Python's
float is the same IEEE binary64 with correctly rounded * and /, as the device's.
"""
import random

import pytest


def weight_before(v, first, wf, ws):
    return wf * v if v <= first else wf * first + ws * (v - first)


def start_fp64(total, v, first, nv, wf, ws):
    wt = weight_before(nv, first, wf, ws)
    return int(float(total) * float(weight_before(v, first, wf, ws)) / float(wt))


def holding_fp64(total, u, first, nv, wf, ws):
    wt = weight_before(nv, first, wf, ws)
    w = int((float(u + 1) * float(wt) - 1.0) / float(total))
    v = w // wf if w < wf * first else first + (w - wf * first) // ws
    return min(v, nv - 1)


SHAPES = [  # (grid, waves per workgroup, workgroups dispatched first, weights)
    (512, 4, 256, (6, 5)), (512, 1, 256, (6, 5)), (512, 4, 256, (1, 1)), (300, 2, 256, (6, 5)),
    (256, 4, 256, (6, 5)), (7, 4, 7, (6, 5)),
]


@pytest.mark.parametrize("grid,wph,first_wgs,weights", SHAPES)
def test_starts_are_exact_floors(grid, wph, first_wgs, weights):
    wf, ws = weights
    nv, first = grid * wph, first_wgs * wph
    wt = weight_before(nv, first, wf, ws)
    rng = random.Random(grid * 31 + wph)
    totals = [1, 2, nv - 1, nv, nv + 1, 131072, 2**31 - 1, 2**36 - 1]
    totals += [rng.randrange(1, 2**36) for _ in range(20)]
    for total in totals:
        vs = list(range(0, min(nv, 64) + 1)) + [first - 1, first, first + 1, nv - 1, nv]
        vs += [rng.randrange(0, nv + 1) for _ in range(64)]
        for v in vs:
            if 0 <= v <= nv:
                exact = total * weight_before(v, first, wf, ws) // wt
                assert start_fp64(total, v, first, nv, wf, ws) == exact, (total, v)
        assert start_fp64(total, 0, first, nv, wf, ws) == 0
        assert start_fp64(total, nv, first, nv, wf, ws) == total


@pytest.mark.parametrize("grid,wph,first_wgs,weights", SHAPES)
def test_holding_inverts_start(grid, wph, first_wgs, weights):
    """holding(u) is the last range whose start is <= u, i.e. the one that processes u."""
    wf, ws = weights
    nv, first = grid * wph, first_wgs * wph
    rng = random.Random(7 + grid)
    for total in [1, 3, nv // 3 + 1, nv, 5 * nv + 17, 131072, 2**36 - 1]:
        starts = [total * weight_before(v, first, wf, ws) // weight_before(nv, first, wf, ws)
                  for v in range(nv + 1)]
        us = set(range(0, min(total, 2000)))
        for v in rng.sample(range(nv), min(nv, 200)):  # units around range boundaries
            for d in (-1, 0, 1):
                if 0 <= starts[v] + d < total:
                    us.add(starts[v] + d)
        us.add(total - 1)
        for u in sorted(us):
            v = holding_fp64(total, u, first, nv, wf, ws)
            assert starts[v] <= u < starts[v + 1], (total, u, v)
