"""Restatement of MLX's affine quantizer in numpy (fp32 arithmetic). TEST INFRASTRUCTURE ONLY.

Reference: mlx-lm's QuantizedKVCache.update_and_fetch and KVCache.to_quantized call
``mx.quantize(x, group_size, bits)`` on every K/V row they store; m5engine/attention.py:106-112
(safe_maybe_quantize_kv_cache) and :66-69/:87-90 (quantized_matmul over the triples) consume the
result. mlx (>= 0.32.4, requirements.txt:3 -- a lower bound, so not pinned) is a third-party
dependency absent from /root/reference and from this container; its CPU quantizer is restated
here from its published algorithm:

  per group of `group_size` consecutive elements (fp32 arithmetic, IEEE round-to-nearest-even):
    xmax, xmin = max, min of float(x)
    n     = 2^bits - 1
    neg   = |xmin| > |xmax|
    s     = max((xmax - xmin) / n, 1e-7);  s = s if neg else -s
    edge  = xmin if neg else xmax
    q0    = rint(edge / s)
    if q0 != 0: s = edge / q0; b = edge  else: b = 0
    code  = clip(rint((x - b) / s), 0, n)      # fp32 s and b, before rounding to T
    store scale = T(s), bias = T(b)            # T = the input dtype, round to nearest even
  pack: word w holds codes w*(32/bits) .. as bits [k*bits, (k+1)*bits), least significant first

Storage conventions of this module: half-precision arrays are carried as their uint16 bit
patterns plus a dtype name ("float16" | "bfloat16"), since numpy has no bfloat16.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32


# ---------------------------------------------------------------- half-precision storage
def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round fp32 to bfloat16 (nearest even); NaN stays NaN."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def to_bits(x: np.ndarray, dtype: str) -> np.ndarray:
    """fp32 values -> uint16 storage of `dtype` (round to nearest even)."""
    if dtype == "float16":
        return f32_to_f16_bits(x)
    if dtype == "bfloat16":
        return f32_to_bf16_bits(x)
    raise ValueError(dtype)


def from_bits(bits: np.ndarray, dtype: str) -> np.ndarray:
    """uint16 storage of `dtype` -> exact fp32 values."""
    if dtype == "float16":
        return f16_bits_to_f32(bits)
    if dtype == "bfloat16":
        return bf16_bits_to_f32(bits)
    raise ValueError(dtype)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round fp32 values to `dtype` and return them as fp32."""
    return from_bits(to_bits(x, dtype), dtype)


# ---------------------------------------------------------------- the quantizer
def group_params(x: np.ndarray, bits: int):
    """Per-group fp32 (scale, bias) before rounding; x is fp32 [..., G]."""
    x = np.asarray(x, np.float32)
    n = F32((1 << bits) - 1)
    xmax = x.max(axis=-1)
    xmin = x.min(axis=-1)
    neg = np.abs(xmin) > np.abs(xmax)
    s = np.maximum((xmax - xmin) / n, F32(1e-7)).astype(np.float32)
    s = np.where(neg, s, -s).astype(np.float32)
    edge = np.where(neg, xmin, xmax).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        q0 = np.rint(edge / s).astype(np.float32)
        nz = q0 != 0
        s = np.where(nz, (edge / np.where(nz, q0, F32(1))).astype(np.float32), s).astype(np.float32)
    b = np.where(nz, edge, F32(0)).astype(np.float32)
    return s, b


def quantize_values(x: np.ndarray, group_size: int = 64, bits: int = 8):
    """fp32 values [..., D] -> (codes uint8-valued uint32 [..., D], s fp32 [..., D/G], b fp32)."""
    x = np.asarray(x, np.float32)
    D = x.shape[-1]
    if D % group_size:
        raise ValueError("D must be a multiple of group_size")
    xg = x.reshape(*x.shape[:-1], D // group_size, group_size)
    s, b = group_params(xg, bits)
    n = F32((1 << bits) - 1)
    with np.errstate(divide="ignore", invalid="ignore"):
        c = np.rint((xg - b[..., None]) / s[..., None]).astype(np.float32)
    c = np.clip(c, F32(0), n).astype(np.uint32)
    return c.reshape(x.shape), s, b


def pack(codes: np.ndarray, bits: int) -> np.ndarray:
    """Codes [..., D] (< 2^bits) -> uint32 [..., D*bits/32], least significant code first."""
    per = 32 // bits
    c = np.asarray(codes, np.uint32)
    c = c.reshape(*c.shape[:-1], c.shape[-1] // per, per)
    shifts = (np.arange(per, dtype=np.uint32) * bits).astype(np.uint32)
    return np.bitwise_or.reduce(c << shifts, axis=-1).astype(np.uint32)


def unpack(words: np.ndarray, bits: int) -> np.ndarray:
    per = 32 // bits
    w = np.asarray(words, np.uint32)[..., None]
    shifts = (np.arange(per, dtype=np.uint32) * bits).astype(np.uint32)
    c = (w >> shifts) & np.uint32((1 << bits) - 1)
    return c.reshape(*w.shape[:-2], w.shape[-2] * per)


def quantize(x_bits: np.ndarray, dtype: str, group_size: int = 64, bits: int = 8):
    """mx.quantize restated: T rows (uint16 storage) -> (codes u32, scales u16, biases u16)."""
    x = from_bits(x_bits, dtype)
    c, s, b = quantize_values(x, group_size, bits)
    return pack(c, bits), to_bits(s, dtype), to_bits(b, dtype)


def dequantize(codes: np.ndarray, scales_bits: np.ndarray, biases_bits: np.ndarray, dtype: str,
               group_size: int = 64, bits: int = 8) -> np.ndarray:
    """Exact dequantization in fp64: scale * code + bias with the stored T scale and bias."""
    c = unpack(codes, bits).astype(np.float64)
    s = from_bits(scales_bits, dtype).astype(np.float64)
    b = from_bits(biases_bits, dtype).astype(np.float64)
    D = c.shape[-1]
    cg = c.reshape(*c.shape[:-1], D // group_size, group_size)
    return (cg * s[..., None] + b[..., None]).reshape(c.shape)


def range_exponent(scales_bits: np.ndarray, biases_bits: np.ndarray, dtype: str, bits: int) -> int:
    """The range exponent of a quantized cache (include/kvq.h, kvq_qtensor.range_exp): the smallest
    E >= 0 with max(|b|, |b + n s|) <= 2^15 * 2^E over every group (n = 2^bits - 1; the group's
    dequantized values s * c + b, c in [0, n], have their extremes at c = 0 and c = n), from the
    stored T scale and bias in fp32 (b + n s rounded after the product, then after the sum). An
    unbounded group (inf) gives 127. No counterpart in the reference: it is this build's operand
    range, and the checks are its defining inequality at the boundaries."""
    s = from_bits(scales_bits, dtype).astype(np.float32)
    b = from_bits(biases_bits, dtype).astype(np.float32)
    if s.size == 0:
        return 0
    top = (b + (np.float32((1 << bits) - 1) * s).astype(np.float32)).astype(np.float32)
    bound = float(np.nan_to_num(np.maximum(np.abs(b), np.abs(top)), nan=0.0, posinf=np.inf).max())
    if bound <= 32768.0:
        return 0
    if not np.isfinite(bound):
        return 127
    e = 0
    while bound > 32768.0 * 2.0**e:
        e += 1
    return e
