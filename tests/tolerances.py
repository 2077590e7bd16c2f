"""Parity bars for attention outputs against the float64 oracle.

bf16 kernels: max-abs <= 2e-2 and mean-abs <= 2e-3 (fp32 softmax/accumulation,
bf16 inputs and output).  fp32 kernels: max-abs <= 1e-5.  KV-cache writes are
compared bit for bit.
"""
from __future__ import annotations

import numpy as np
import torch

BF16_MAX_ABS = 2e-2
BF16_MEAN_ABS = 2e-3
F32_MAX_ABS = 1e-5


def to_np(t) -> np.ndarray:
    if isinstance(t, torch.Tensor):
        return t.detach().float().cpu().numpy().astype(np.float64) if t.dtype != torch.float64 \
            else t.detach().cpu().numpy()
    return np.asarray(t, dtype=np.float64)


def errors(out, ref):
    d = np.abs(to_np(out) - to_np(ref))
    return float(d.max()) if d.size else 0.0, float(d.mean()) if d.size else 0.0


def assert_attn_close(out, ref, dtype, what: str = "") -> None:
    mx, mean = errors(out, ref)
    assert np.all(np.isfinite(to_np(out))), f"{what}: non-finite output"
    if dtype == torch.float32:
        assert mx <= F32_MAX_ABS, f"{what}: max-abs {mx:.3g} > {F32_MAX_ABS}"
    else:
        assert mx <= BF16_MAX_ABS and mean <= BF16_MEAN_ABS, (
            f"{what}: max-abs {mx:.3g} (bar {BF16_MAX_ABS}), mean-abs {mean:.3g} "
            f"(bar {BF16_MEAN_ABS})")
