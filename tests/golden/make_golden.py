"""Write the golden fixtures of tests/golden/ from the oracle (run on CPU).

Inputs are regenerated from seeds by nano_inference_amd.workloads on the CPU
(torch's CPU generator is deterministic); each fixture stores the sha256 of
its inputs so a test can tell generator drift from a kernel regression, and
the oracle's float64 output stored as float32.

Usage: python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from nano_inference_amd import workloads  # noqa: E402
from oracle import reference_attention as ref  # noqa: E402
from oracle import textbook as tb  # noqa: E402


def digest(*tensors) -> str:
    h = hashlib.sha256()
    for t in tensors:
        h.update(t.contiguous().view(torch.uint8).numpy().tobytes())
    return h.hexdigest()


# name -> builder returning (inputs digest, expected float64 array)
def decode_small_f32():
    c = workloads.decode_small("cpu", torch.float32)
    kc, vc = c.k_cache[0].clone(), c.v_cache[0].clone()
    ref.kv_write_loop(c.k_new, c.v_new, kc, vc, c.slot_mapping)
    out = tb.paged_decode(c.q.double().numpy(), kc.double().numpy(), vc.double().numpy(),
                          c.block_tables.numpy(), c.context_lens.numpy(), 1 / math.sqrt(128))
    return digest(c.q, c.k_new, c.v_new, c.k_cache, c.v_cache), out


def decode_small_bf16():
    c = workloads.decode_small("cpu", torch.bfloat16)
    kc, vc = c.k_cache[0].clone(), c.v_cache[0].clone()
    ref.kv_write_loop(c.k_new, c.v_new, kc, vc, c.slot_mapping)
    out = tb.paged_decode(c.q.double().numpy(), kc.double().numpy(), vc.double().numpy(),
                          c.block_tables.numpy(), c.context_lens.numpy(), 1 / math.sqrt(128))
    return digest(c.q, c.k_new, c.v_new, c.k_cache, c.v_cache), out


def varlen_causal_small():
    c = workloads.make_varlen([3, 17, 40], 4, 2, 128, torch.bfloat16, "cpu", 606, True)
    cu = c.cu_seqlens.numpy()
    res = tb.varlen(c.q.double().numpy(), c.k.double().numpy(), c.v.double().numpy(), cu[:-1],
                    np.diff(cu), cu[:-1], np.diff(cu), 1 / math.sqrt(128), "top_left")
    out = np.concatenate([res[s][1] for s in range(len(c.lens))])
    return digest(c.q, c.k, c.v), out


def vision_window_small():
    from nano_inference_amd.vision import window_index
    cu = window_index([(1, 8, 12)])[1]
    lens = [int(b - a) for a, b in zip(cu[:-1], cu[1:])]
    c = workloads.make_varlen(lens, 2, 2, 80, torch.bfloat16, "cpu", 707, False)
    cuv = c.cu_seqlens.numpy()
    res = tb.varlen(c.q.double().numpy(), c.k.double().numpy(), c.v.double().numpy(), cuv[:-1],
                    np.diff(cuv), cuv[:-1], np.diff(cuv), 1 / math.sqrt(80), "none")
    out = np.concatenate([res[s][1] for s in range(len(c.lens))])
    return digest(c.q, c.k, c.v), out


def chunked_small():
    c = workloads.chunked_qwen3_8b("cpu", n=2, chunk=24, prior=[40, 3], seed=808, num_heads=4,
                                  num_kv_heads=2)
    res = tb.paged_prefill(c.q.double().numpy(), c.k_cache.double().numpy(),
                           c.v_cache.double().numpy(), c.block_tables.numpy(),
                           c.q_start.numpy(), c.q_len.numpy(), c.context_lens.numpy(),
                           1 / math.sqrt(128), "bottom_right")
    out = np.concatenate([res[s][1] for s in range(2)])
    return digest(c.q, c.k_cache, c.v_cache), out


FIXTURES = {
    "decode_small_f32": decode_small_f32,
    "decode_small_bf16": decode_small_bf16,
    "varlen_causal_small": varlen_causal_small,
    "vision_window_small": vision_window_small,
    "chunked_small": chunked_small,
}


def main():
    for name, fn in FIXTURES.items():
        dig, out = fn()
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, out=out.astype(np.float32), digest=np.array(dig))
        print(f"{path}: {out.shape} {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
