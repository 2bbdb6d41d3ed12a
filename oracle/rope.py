"""Restatement of rotary position embedding (RoPE) in numpy. TEST INFRASTRUCTURE ONLY.

Reference: mlx-lm's attention layers rotate queries and keys with nn.RoPE(dims, traditional,
base, scale) (mx.fast.rope; third-party, absent here) before the cache update. The reference's
native engine fuses the split-half ("NeoX", mlx traditional=False) rotation with the KV write at
native/src/kernels.metal:106-160:

    freq  = 1 / pow(theta, 2d / head_dim);   angle = pos * freq
    x[d]        = x0 * cos - x1 * sin
    x[d + half] = x1 * cos + x0 * sin

This module follows that kernel for the split-half pairs, adds the interleaved pairs (2i, 2i + 1)
of traditional=True and nn.RoPE's position scale and partial `dims`, and fixes the numerics the
GPU kernel implements:

    freq_i   = fp32(1 / base^(2i / dims))          evaluated in double precision, then rounded
    angle    = fp32(fp32(pos * scale) * freq_i)
    cos, sin = fp32 of the double-precision cos / sin of that fp32 angle
    products and sums in fp32, not fused; the result rounded to T

MLX-exactness is parity unpinned: mx.fast.rope does not run here. The GPU kernel's fp32 sincos is
within about one ulp of the correctly rounded values used here, which moves a rounded T value by
one ulp in rare cases; tests/test_gpu_rope.py states that tolerance.
"""

from __future__ import annotations

import numpy as np

from . import quantize as OQ

F32 = np.float32


def freqs(dims: int, base: float) -> np.ndarray:
    """fp32 frequency of each of the dims / 2 pairs."""
    i = np.arange(dims // 2, dtype=np.float64)
    return (1.0 / np.power(float(F32(base)), 2.0 * i / dims)).astype(F32)


def angles(positions: np.ndarray, dims: int, base: float, scale: float) -> np.ndarray:
    """fp32 angle [len(positions), dims / 2]."""
    p = (np.asarray(positions, dtype=np.int64).astype(F32) * F32(scale)).astype(F32)
    return (p[:, None] * freqs(dims, base)[None, :]).astype(F32)


def rope_f32(x: np.ndarray, dims: int, traditional: bool, base: float, scale: float, offset: int) -> np.ndarray:
    """Rotate fp32 x [..., L, D] (row l at position offset + l); returns fp32, not yet rounded."""
    x = np.asarray(x, dtype=F32)
    L = x.shape[-2]
    ang = angles(offset + np.arange(L), dims, base, scale).astype(np.float64)
    c, s = np.cos(ang).astype(F32), np.sin(ang).astype(F32)  # [L, dims / 2]
    out = x.copy()
    if traditional:
        a, b = x[..., 0:dims:2], x[..., 1:dims:2]
        out[..., 0:dims:2] = (a * c).astype(F32) - (b * s).astype(F32)
        out[..., 1:dims:2] = (a * s).astype(F32) + (b * c).astype(F32)
    else:
        h = dims // 2
        a, b = x[..., :h], x[..., h:dims]
        out[..., :h] = (a * c).astype(F32) - (b * s).astype(F32)
        out[..., h:dims] = (b * c).astype(F32) + (a * s).astype(F32)
    return out.astype(F32)


def rope(x_bits: np.ndarray, dtype: str, dims: int, traditional: bool, base: float, scale: float,
         offset: int) -> np.ndarray:
    """RoPE of half-precision rows given as bit patterns; returns the rounded result's bits."""
    y = rope_f32(OQ.from_bits(x_bits, dtype), dims, traditional, base, scale, offset)
    return OQ.to_bits(y, dtype)


def rope_quantize(x_bits: np.ndarray, dtype: str, group_size: int, bits: int, dims: int, traditional: bool,
                  base: float, scale: float, offset: int):
    """What the fused rotate-and-quantize append stores: RoPE, round to T, then mx.quantize."""
    return OQ.quantize(rope(x_bits, dtype, dims, traditional, base, scale, offset), dtype, group_size, bits)
