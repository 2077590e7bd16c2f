"""ViT chunk producers: the oracle restatement, the package's producers and invariants.

Grids of the vision workload: (1,28,28), (1,36,52), (1,64,48), (1,20,90) patches;
window 112 px / merge 2 / patch 14 -> 4x4 merge groups = up to 64 patches.
"""
import numpy as np

from nano_inference_amd import full_cu_seqlens, window_index
from nano_inference_amd.workloads import VISION_GRIDS
from oracle import vision_windows as vw


def test_window_counts_for_the_workload_grids():
    wi, cu = vw.get_window_index(VISION_GRIDS)
    lens = np.diff(cu.numpy())
    assert int(cu[-1]) == 784 + 1872 + 3072 + 1800 == 7528
    assert len(lens) == 135
    assert lens.max() == 64 and lens.min() >= 4 and (lens % 4 == 0).all()
    assert sorted(wi.tolist()) == list(range(7528 // 4))


def test_package_producers_equal_restatement():
    for grids in (VISION_GRIDS, [(2, 8, 12)], [(1, 14, 6), (3, 4, 4)]):
        wi, cu = vw.get_window_index(grids)
        pw, pc = window_index(grids)
        assert pw.tolist() == wi.tolist()
        assert pc.tolist() == cu.tolist()
        assert full_cu_seqlens(grids).tolist() == vw.full_cu_seqlens(grids).tolist()


def test_windows_equal_bruteforce_enumeration():
    """Every window is the set of 4x4 merge groups of one frame, clipped at the edge."""
    for grids in (VISION_GRIDS, [(2, 10, 6)]):
        wi, cu = vw.get_window_index(grids)
        wi = wi.tolist()
        expect, off = [], 0
        for t, h, w in grids:
            gh, gw = h // 2, w // 2
            for ti in range(t):
                for y0 in range(0, gh, 4):
                    for x0 in range(0, gw, 4):
                        expect.append([off + ti * gh * gw + y * gw + x
                                       for y in range(y0, min(y0 + 4, gh))
                                       for x in range(x0, min(x0 + 4, gw))])
            off += t * gh * gw
        got = [wi[a // 4:b // 4] for a, b in zip(cu[:-1].tolist(), cu[1:].tolist())]
        assert got == expect


def test_full_cu_seqlens():
    assert vw.full_cu_seqlens(VISION_GRIDS).tolist() == [0, 784, 2656, 5728, 7528]
    assert vw.full_cu_seqlens([(2, 4, 6)]).tolist() == [0, 24, 48]
