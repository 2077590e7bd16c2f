"""fp8 KV-cache format and its write loop (oracle).

TEST INFRASTRUCTURE ONLY: imported by tests, never by the product.

The reference keeps K/V in the model dtype (src/nano_inference/kv_cache/allocator.py:
35-39).  The fp8 variant stores every (token, KV head) row of D values as OCP
float8 e4m3 (torch.float8_e4m3fn: 4 exponent bits, bias 7, 3 mantissa bits, max
448, no infinities) with one float32 scale per row:

    scale = max_d |x_d| / 448          (fp32, correctly rounded)
    code_d = e4m3(x_d / scale)         (fp32 division, round to nearest even)
    x_d ~= float(code_d) * scale

A row of zeros stores scale 0 and zero codes.  The row's largest magnitude maps
to +-448 exactly, so no code saturates.  Scales live in [num_blocks, H_kv, BS]
float32 tensors beside the caches; the write follows the reference's per-token
loop (src/nano_inference/layers/attention.py:267-278) with the quantisation
applied to each row.
"""
from __future__ import annotations

import torch

E4M3_MAX = 448.0


def e4m3_value(code: int) -> float:
    """Value of an e4m3fn code from the format's definition (NaN for 0x7F / 0xFF)."""
    s = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 0xF
    m = code & 0x7
    if e == 0xF and m == 0x7:
        return float("nan")
    if e == 0:
        return s * (m / 8.0) * 2.0 ** -6
    return s * (1.0 + m / 8.0) * 2.0 ** (e - 7)


def quantize_rows(x: torch.Tensor):
    """Rows (..., D) of any float dtype -> (codes uint8 (..., D), scales float32 (...))."""
    xf = x.float()
    amax = xf.abs().amax(dim=-1)
    scale = amax / E4M3_MAX
    safe = torch.where(scale > 0, scale, torch.ones_like(scale))
    q = (xf / safe.unsqueeze(-1)).to(torch.float8_e4m3fn)
    q = torch.where((scale > 0).unsqueeze(-1), q.view(torch.uint8),
                    torch.zeros_like(q.view(torch.uint8)))
    return q, scale


def dequantize_rows(codes: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """(..., D) uint8 codes and (...) scales -> float32 rows."""
    return codes.view(torch.float8_e4m3fn).float() * scales.unsqueeze(-1)


def kv_write_loop_fp8(k, v, k_cache, v_cache, k_scale, v_scale, slot_mapping) -> None:
    """The reference's write loop (attention.py:267-278) into the fp8 format.

    k, v (B, S, H_kv, D); caches [NB, H_kv, BS, D] uint8; scales [NB, H_kv, BS] fp32;
    slot_mapping (B, S) int64, negative = skip.
    """
    bs = k_cache.shape[2]
    for b in range(k.shape[0]):
        for s in range(k.shape[1]):
            slot = int(slot_mapping[b, s])
            if slot < 0:
                continue
            qk, sk = quantize_rows(k[b, s])
            qv, sv = quantize_rows(v[b, s])
            k_cache[slot // bs, :, slot % bs, :] = qk
            v_cache[slot // bs, :, slot % bs, :] = qv
            k_scale[slot // bs, :, slot % bs] = sk
            v_scale[slot // bs, :, slot % bs] = sv
