"""FP8 KV cache rows for :func:`dsa_amd.forward` (no reference counterpart: the
reference takes a contiguous bf16 cache only, dsa/api.py:30-33).

One row per token, 656 bytes -- the layout of DeepSeek-V3.2's FP8 MLA cache:

* bytes   0..511: the 512 latent values as OCP float8 e4m3 (bias 7, max 448),
* bytes 512..527: 4 fp32 scales, scale i for dims 128 i .. 128 i + 127,
* bytes 528..655: the 64 rope values as bf16 (not quantized).

The attention kernels compute with ``bf16(fp32(e4m3) * scale)`` for the latent
values, for any positive scale; with power-of-two scales (2^-100 .. 2^100)
that value is exact and they expand the rows with one conversion
instruction per two values.  :func:`quantize_kv_fp8` writes such rows from a
bf16 cache: per 128-dim block the scale is the smallest power of two with
``amax / scale <= 448`` (e4m3 is floating point, so a power-of-two scale
costs no relative precision), or exactly ``amax / 448`` with
``pow2_scales=False``.  It is ordinary tensor code (the cache writer sits
outside the attention's hot path).
"""
from __future__ import annotations

import torch

FP8_ROW = 656
E4M3_MAX = 448.0


def quantize_kv_fp8(kv, k_rope, pow2_scales: bool = True):
    """``kv [..., 512]`` bf16 and ``k_rope [..., 64]`` bf16 (same leading dims)
    -> uint8 rows ``[..., 656]`` on the same device."""
    if kv.shape[-1] != 512 or k_rope.shape[-1] != 64 or kv.shape[:-1] != k_rope.shape[:-1]:
        raise ValueError("expected kv[..., 512] and k_rope[..., 64] with the same leading dims")
    if kv.dtype != torch.bfloat16 or k_rope.dtype != torch.bfloat16:
        raise ValueError("kv and k_rope must be bfloat16")
    lead = kv.shape[:-1]
    x = kv.float().reshape(*lead, 4, 128)
    amax = x.abs().amax(-1, keepdim=True)
    scale = torch.where(amax > 0, amax / E4M3_MAX, torch.ones_like(amax))
    if pow2_scales:  # the smallest power of two >= amax / 448: frexp gives s = m 2^e, m in [0.5, 1)
        m, e = torch.frexp(scale)
        scale = torch.ldexp(torch.ones_like(scale), e - (m == 0.5).to(e.dtype))
    codes = (x / scale).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn).reshape(*lead, 512)
    rows = torch.cat([codes.view(torch.uint8),
                      scale.reshape(*lead, 4).contiguous().view(torch.uint8),
                      k_rope.contiguous().view(torch.uint8)], dim=-1)
    return rows.contiguous()
