"""Host plan of continuous batching with chunked prefill (nano_inference_amd.e2e.ChunkedScheduler).

Simulated on the CPU over seeded prompt lengths: every prompt position is fed
exactly once and in order, decode positions continue the prompt one token per step,
every sequence samples tokens 0 .. max_new - 1 exactly once and in order, each
step holds at most max_step_tokens tokens with the decodes first, no chunk exceeds
the chunk size, and every sequence is admitted and leaves exactly once.
"""
import random

import pytest

from nano_inference_amd.e2e import ChunkedScheduler


@pytest.mark.parametrize("seed,max_new,step_tokens,chunk", [
    (0, 256, 4096, 512), (1, 1, 4096, 512), (2, 7, 300, 64), (3, 3, 64, 1000), (4, 20, 9, 4)])
def test_plan_invariants(seed, max_new, step_tokens, chunk):
    rng = random.Random(seed)
    lens = [rng.randint(1, 2048 if step_tokens > 1000 else 200) for _ in range(rng.randint(1, 64))]
    admitted, left = [], []
    sched = ChunkedScheduler(lens, max_new, step_tokens, chunk, admitted.append, left.append)
    fed = {i: [] for i in range(len(lens))}
    samples = {i: [] for i in range(len(lens))}
    steps = 0
    while not sched.done():
        step = sched.plan()
        assert step, "a step with work left must carry tokens"
        assert sum(e.n for e in step) <= max(step_tokens, sum(e.decode for e in step))
        kinds = [e.decode for e in step]
        assert kinds == sorted(kinds, reverse=True), "decodes first"
        for e in step:
            assert e.sid in admitted and e.sid not in left
            if e.decode:
                assert e.n == 1
            else:
                assert 1 <= e.n <= chunk
            fed[e.sid].extend(range(e.start, e.start + e.n))
            if e.sample is not None:
                samples[e.sid].append(e.sample)
        sched.commit(step)
        steps += 1
        assert steps < 100000
    assert sorted(admitted) == list(range(len(lens))) == sorted(left)
    for i, n in enumerate(lens):
        assert fed[i] == list(range(n + max_new - 1)), i
        assert samples[i] == list(range(max_new)), i
