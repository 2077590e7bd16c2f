"""The unit ranges of the split decode kernel, as its fp64 arithmetic forms them.

Virtual wave v of V (workgroup v >> wl, 2^wl virtual waves per workgroup) owns units
[start(v), start(v + 1)) with start(v) = floor(total * W(v) / W(V)), W(v) summing the
weights of the virtual waves before v; each weighs its workgroup's class weight: first or
second dispatched on its CU (below or above `first` workgroups) and even or odd workgroup
index (the XCD it runs on).  The kernel evaluates the quotient in fp64, which is exact only
while the products stay below 2^53 and a non-integer quotient lies further from an integer
than the rounding error.  The host refuses batches of more than 2^36 units, so these checks
run up to that size: Python's float is the same IEEE binary64 with correctly rounded * and
/, as the device's.  The weights are the kernel's bf16 table (13, 12, 11, 10); over the fp8
format the ranges are even (W(v) = v).  The closed forms the kernel uses are checked against
plain sums.  The merge kernel does no range arithmetic: the split kernel records the ranges
that hold each sequence (checked on the GPU by the decode tests).
"""
import random

import pytest

BF16_WEIGHTS = (13, 12, 11, 10)  # first even, first odd, second even, second odd


def wg_weight(i, first, w):
    return (w[1] if i & 1 else w[0]) if i < first else (w[3] if i & 1 else w[2])


def wg_sum(n, first, w):
    """Closed form of sum(wg_weight(i) for i < n), as the kernel computes it."""
    n1 = min(n, first)
    s = w[0] * ((n1 + 1) >> 1) + w[1] * (n1 >> 1)
    if n > first:
        s += w[2] * (((n + 1) >> 1) - ((first + 1) >> 1)) + w[3] * ((n >> 1) - (first >> 1))
    return s


def weight_before(v, first, wl, w):
    if w is None:  # fp8: even ranges
        return v
    n = v >> wl
    s = v - (n << wl)
    return (wg_sum(n, first, w) << wl) + s * wg_weight(n, first, w)


def start_fp64(total, v, first, wl, nv, w):
    wt = weight_before(nv, first, wl, w)
    return int(float(total) * float(weight_before(v, first, wl, w)) / float(wt))


SHAPES = [  # (grid, log2 waves per workgroup, workgroups dispatched first, weights)
    (512, 0, 256, BF16_WEIGHTS), (512, 2, 256, BF16_WEIGHTS), (512, 1, 256, BF16_WEIGHTS),
    (512, 2, 256, None), (300, 1, 256, BF16_WEIGHTS), (256, 2, 256, BF16_WEIGHTS),
    (7, 2, 7, BF16_WEIGHTS), (301, 0, 255, BF16_WEIGHTS), (40, 1, 17, BF16_WEIGHTS),
]


@pytest.mark.parametrize("grid,wl,first_wgs,weights", [s for s in SHAPES if s[3] is not None])
def test_closed_forms_match_plain_sums(grid, wl, first_wgs, weights):
    for n in range(grid + 1):
        assert wg_sum(n, first_wgs, weights) == sum(
            wg_weight(i, first_wgs, weights) for i in range(n))
    nv = grid << wl
    acc = 0
    for v in range(nv + 1):
        assert weight_before(v, first_wgs, wl, weights) == acc, v
        if v < nv:
            acc += wg_weight(v >> wl, first_wgs, weights)
    assert weight_before(nv, first_wgs, wl, weights) < 2**15


@pytest.mark.parametrize("grid,wl,first_wgs,weights", SHAPES)
def test_starts_are_exact_floors(grid, wl, first_wgs, weights):
    nv = grid << wl
    wt = weight_before(nv, first_wgs, wl, weights)
    rng = random.Random(grid * 31 + wl)
    totals = [1, 2, nv - 1, nv, nv + 1, 131072, 2**31 - 1, 2**36 - 1]
    totals += [rng.randrange(1, 2**36) for _ in range(20)]
    first = first_wgs << wl
    for total in totals:
        vs = list(range(0, min(nv, 64) + 1)) + [first - 1, first, first + 1, nv - 1, nv]
        vs += [rng.randrange(0, nv + 1) for _ in range(64)]
        for v in vs:
            if 0 <= v <= nv:
                exact = total * weight_before(v, first_wgs, wl, weights) // wt
                assert start_fp64(total, v, first_wgs, wl, nv, weights) == exact, (total, v)
        assert start_fp64(total, 0, first_wgs, wl, nv, weights) == 0
        assert start_fp64(total, nv, first_wgs, wl, nv, weights) == total


@pytest.mark.parametrize("grid,wl,first_wgs,weights", SHAPES)
def test_ranges_tile_the_units_in_order(grid, wl, first_wgs, weights):
    """Consecutive ranges meet (no unit is skipped or taken twice) and a range's length
    follows its class weight to within one unit."""
    nv = grid << wl
    for total in [3, nv, 7 * nv + 5, 131072]:
        starts = [start_fp64(total, v, first_wgs, wl, nv, weights) for v in range(nv + 1)]
        assert starts[0] == 0 and starts[-1] == total
        assert all(a <= b for a, b in zip(starts, starts[1:]))
        wt = weight_before(nv, first_wgs, wl, weights)
        for v in range(nv):
            w = 1 if weights is None else wg_weight(v >> wl, first_wgs, weights)
            assert abs((starts[v + 1] - starts[v]) - total * w / wt) < 1.0 + 1e-9


def test_a_planted_mistake_fails():
    """Swapping the odd and even weights of the second half moves range starts, which the
    exact-floor check above would catch in a kernel that paired the classes the other way."""
    grid, wl, first = 512, 2, 256
    nv = grid << wl
    swapped = (BF16_WEIGHTS[0], BF16_WEIGHTS[1], BF16_WEIGHTS[3], BF16_WEIGHTS[2])
    a = [start_fp64(131072, v, first, wl, nv, BF16_WEIGHTS) for v in range(nv + 1)]
    b = [start_fp64(131072, v, first, wl, nv, swapped) for v in range(nv + 1)]
    assert a != b
