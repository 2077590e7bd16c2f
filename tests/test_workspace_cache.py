"""The decode workspace cache of ops.decode_workspace: one buffer per (device, stream),
reused by later calls on that stream, a fresh one for another stream, and a buffer that
is outgrown kept alive (a captured HIP graph may still hold its address) rather than freed,
geometric growth so that the kept ones add up to less than the live one, and their release.

Runs on the CPU: the cache keys on ``stream.cuda_stream`` and allocates on the device it
is given, so CPU tensors and stand-in stream objects exercise the same code.
"""
import gc
import weakref

import pytest
import torch

from nano_inference_amd import ops


class _Stream:
    def __init__(self, handle):
        self.cuda_stream = handle


@pytest.fixture(autouse=True)
def _clean_cache():
    saved_ws, saved_retired = dict(ops._DECODE_WS), list(ops._RETIRED)
    ops._DECODE_WS.clear()
    ops._RETIRED.clear()
    yield
    ops._DECODE_WS.clear()
    ops._DECODE_WS.update(saved_ws)
    ops._RETIRED[:] = saved_retired


def test_one_workspace_per_stream_reused_by_later_calls():
    dev = torch.device("cpu")
    s1, s2 = _Stream(0x1000), _Stream(0x2000)
    a = ops.decode_workspace(dev, 4096, stream=s1)
    assert a.numel() >= 4096 and a.dtype == torch.uint8
    assert ops.decode_workspace(dev, 100, stream=s1).data_ptr() == a.data_ptr()
    b = ops.decode_workspace(dev, 4096, stream=s2)
    assert b.data_ptr() != a.data_ptr(), "two streams must not share work memory"
    assert ops.decode_workspace(dev, 4096, stream=s2).data_ptr() == b.data_ptr()
    assert ops.decode_workspace(dev, 4096, stream=s1).data_ptr() == a.data_ptr()


def test_outgrown_workspace_is_kept_alive_not_freed():
    dev = torch.device("cpu")
    s = _Stream(0x3000)
    small = ops.decode_workspace(dev, 1 << 20, stream=s)
    ptr = small.data_ptr()
    ref = weakref.ref(small)
    del small
    big = ops.decode_workspace(dev, (1 << 20) + 1, stream=s)
    assert big.data_ptr() != ptr and big.numel() >= (1 << 20) + 1
    gc.collect()
    # the old buffer still exists (held by the cache), so an address captured in a graph
    # stays valid
    assert ref() is not None and ref().data_ptr() == ptr
    assert any(t.data_ptr() == ptr for t in ops._RETIRED)
    # and the stream now gets the larger one
    assert ops.decode_workspace(dev, 10, stream=s).data_ptr() == big.data_ptr()


def test_minimum_size_and_distinct_devices_keys():
    s = _Stream(0x4000)
    w = ops.decode_workspace(torch.device("cpu"), 1, stream=s)
    assert w.numel() >= 1 << 20  # small requests get a 1 MiB buffer, so growth is rare
    assert (-1, 0x4000) in ops._DECODE_WS  # (device index, stream handle); -1: not a GPU


def test_growth_is_geometric_and_retired_total_stays_below_the_live_size():
    """A stream whose calls ask for slowly growing sizes (an fp32 serving loop whose
    contexts grow) keeps less in retired workspaces than its live one holds."""
    dev = torch.device("cpu")
    s = _Stream(0x5000)
    need = 1 << 20
    sizes = []
    for _ in range(200):
        need += 123_457  # ~0.12 MB more per call
        ws = ops.decode_workspace(dev, need, stream=s)
        assert ws.numel() >= need
        if not sizes or sizes[-1] != ws.numel():
            sizes.append(ws.numel())
    assert all(b >= 2 * a for a, b in zip(sizes, sizes[1:])), sizes
    assert len(ops._RETIRED) == len(sizes) - 1
    assert ops.retired_workspace_bytes() < sizes[-1]


def test_release_frees_the_retired_workspaces_only():
    dev = torch.device("cpu")
    s = _Stream(0x6000)
    ops.decode_workspace(dev, 1 << 20, stream=s)
    old = weakref.ref(ops._RETIRED[-1]) if ops._RETIRED else None
    live = ops.decode_workspace(dev, 3 << 20, stream=s)
    assert old is None and len(ops._RETIRED) == 1
    ref = weakref.ref(ops._RETIRED[0])
    assert ops.release_retired_workspaces() == 1 << 20
    gc.collect()
    assert ref() is None and ops._RETIRED == []
    assert ops.decode_workspace(dev, 10, stream=s).data_ptr() == live.data_ptr()
