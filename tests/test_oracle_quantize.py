"""Pins the CPU restatement of MLX's affine quantizer (oracle/quantize.py).

Checks chosen so that a plausible slip fails one of them: a wrong sign rule or tie-break
(all-zero / constant / ramp KATs), dividing instead of multiplying or using the rounded scale
(ramp codes, bound on reconstruction), wrong packing order (pack/unpack and hand-packed words),
wrong half-precision rounding (against torch's own conversions), and any divergence between the
numpy and C restatements.
"""

import ctypes
import subprocess
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import quantize as Q

ROOT = Path(__file__).resolve().parents[1]


def _bits(v: float, dtype: str) -> int:
    return int(Q.to_bits(np.array([v], np.float32), dtype)[0])


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("bits", [2, 4, 8])
def test_all_zero_group(dtype, bits):
    x = Q.to_bits(np.zeros((1, 64), np.float32), dtype)
    codes, s, b = Q.quantize(x, dtype, 64, bits)
    assert (codes == 0).all()
    # s = -max(0, 1e-7) stored in T; bias exactly 0
    assert int(s[0, 0]) == _bits(-1e-7, dtype)
    assert int(b[0, 0]) == 0
    if dtype == "float16":
        assert int(s[0, 0]) == 0x8002  # -2 * 2^-24, the f16 subnormal nearest to -1e-7


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("c", [0.5, -3.25, 17.0])
def test_constant_group(dtype, c):
    x = Q.to_bits(np.full((1, 64), c, np.float32), dtype)
    codes, s, b = Q.quantize(x, dtype, 64, 8)
    assert (codes == 0).all()
    assert int(b[0, 0]) == _bits(c, dtype)  # bias = edge = the constant
    xhat = Q.dequantize(codes, s, b, dtype, 64, 8)
    assert np.all(xhat == Q.from_bits(x, dtype))


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("sign", [1, -1])
def test_integer_ramp(dtype, sign):
    """x_j = sign * j, j = 0..63 at 8 bits: |edge| = 63 sits at j = 63 and maps to code 0;
    code_j = round((63 - j) * 255 / 63) exactly (no ties: 255/63 = 85/21 has odd denominator)."""
    x = Q.to_bits(sign * np.arange(64, dtype=np.float32)[None], dtype)
    codes, s, b = Q.quantize(x, dtype, 64, 8)
    c = Q.unpack(codes, 8)[0]
    want = [round(Fraction((63 - j) * 255, 63)) for j in range(64)]
    assert c.tolist() == want
    assert c[0] == 255 and c[63] == 0
    assert int(b[0, 0]) == _bits(sign * 63.0, dtype)
    s_f32 = np.float32(sign * 63.0) / np.float32(-255.0)  # s = edge / q0 with q0 = -255
    assert int(s[0, 0]) == _bits(float(s_f32), dtype)
    assert (s_f32 < 0) == (sign > 0)  # positive-dominant groups get a negative scale


def test_pack_order():
    codes = np.arange(8, dtype=np.uint32)[None]  # 4-bit codes 0..7
    w = Q.pack(codes, 4)
    assert w.tolist() == [[0x76543210]]
    codes8 = np.array([[0x11, 0x22, 0x33, 0x44]], np.uint32)
    assert Q.pack(codes8, 8).tolist() == [[0x44332211]]
    rng = np.random.default_rng(0)
    for bits in (2, 4, 8):
        c = rng.integers(0, 1 << bits, size=(3, 128)).astype(np.uint32)
        assert np.array_equal(Q.unpack(Q.pack(c, bits), bits), c)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_half_rounding_matches_torch(dtype):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(4096) * np.exp(rng.uniform(-30, 30, 4096))).astype(np.float32)
    x = np.concatenate([x, np.array([0.0, -0.0, 1e-40, 65504.0, 65520.0, 1e30], np.float32)])
    tdt = torch.float16 if dtype == "float16" else torch.bfloat16
    ref = torch.from_numpy(x).to(tdt).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(Q.to_bits(x, dtype), ref)
    assert np.array_equal(Q.from_bits(ref, dtype), torch.from_numpy(ref.view(np.int16)).view(tdt).float().numpy())


def _random_groups(rng, rows, D, dtype):
    x = rng.standard_normal((rows, D)).astype(np.float32)
    x[::7] *= 8.0  # outlier rows
    x[3::11, 5] = 40.0  # single outliers
    x[5::13] = np.abs(x[5::13])  # all-positive groups
    x[6::13] = -np.abs(x[6::13])  # all-negative groups
    return Q.to_bits(x, dtype)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("bits,G", [(8, 64), (4, 64), (2, 32), (8, 128), (4, 32)])
def test_properties(dtype, bits, G):
    rng = np.random.default_rng(bits * 1000 + G)
    xb = _random_groups(rng, 257, 128, dtype)
    x = Q.from_bits(xb, dtype)
    c, s, b = Q.quantize_values(x, G, bits)
    n = (1 << bits) - 1
    assert c.min() >= 0 and c.max() <= n
    xg = x.reshape(257, 128 // G, G).astype(np.float64)
    cg = c.reshape(257, 128 // G, G).astype(np.float64)
    xhat = cg * s[..., None].astype(np.float64) + b[..., None].astype(np.float64)
    err = np.abs(xhat - xg)
    half = np.abs(s[..., None]) * (0.5 + 1e-5) + 1e-6 * np.abs(xg)
    # codes strictly inside (0, n) are rounded, so they are within half a step
    inner = (cg > 0) & (cg < n)
    assert np.all(err[inner] <= np.broadcast_to(half, err.shape)[inner])
    # the scale is re-derived from the edge so that 0 is representable (s = edge / rint(edge / s));
    # that can shrink the covered range by up to half a step per code, so a value clipped at code n
    # may miss by up to about one step, never more
    assert np.all(err <= np.abs(s[..., None]) * 1.5 + 1e-6 * np.abs(xg))
    # the larger-magnitude extreme maps to code 0 and reconstructs as the bias
    edge_idx = np.where(np.abs(xg.min(-1)) > np.abs(xg.max(-1)), xg.argmin(-1), xg.argmax(-1))
    ce = np.take_along_axis(cg, edge_idx[..., None], -1)[..., 0]
    assert np.all(ce == 0)
    assert np.all(b == np.take_along_axis(xg, edge_idx[..., None], -1)[..., 0].astype(np.float32))
    # the stored (T-rounded) triple adds at most the rounding of s over n codes and of b
    codes, sb, bb = Q.quantize(xb, dtype, G, bits)
    xq = Q.dequantize(codes, sb, bb, dtype, G, bits).reshape(257, 128 // G, G)
    u = 2.0**-11 if dtype == "float16" else 2.0**-8
    tol = np.abs(s[..., None]) * (np.where(inner, 0.5, 1.5) + n * u) + u * np.abs(b[..., None]) + 1e-7
    assert np.all(np.abs(xq - xg) <= tol)


@pytest.fixture(scope="module")
def cref():
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)
    lib = ctypes.CDLL(str(ROOT / "oracle" / "_build" / "libquant_ref.so"))
    lib.kvq_ref_quantize.restype = None
    return lib


@pytest.mark.parametrize("bits,G", [(8, 64), (4, 64), (2, 32), (4, 128)])
def test_numpy_matches_c_restatement(cref, bits, G):
    rng = np.random.default_rng(7 + bits)
    for dtype in ("float16", "bfloat16"):
        x = Q.from_bits(_random_groups(rng, 513, 128, dtype), dtype)
        c_np, s_np, b_np = Q.quantize_values(x, G, bits)
        rows, D = x.shape
        codes = np.zeros((rows, D * bits // 32), np.uint32)
        s = np.zeros((rows, D // G), np.float32)
        b = np.zeros((rows, D // G), np.float32)
        P = ctypes.POINTER
        cref.kvq_ref_quantize(
            np.ascontiguousarray(x).ctypes.data_as(P(ctypes.c_float)), ctypes.c_size_t(rows), D, G, bits,
            codes.ctypes.data_as(P(ctypes.c_uint32)), s.ctypes.data_as(P(ctypes.c_float)),
            b.ctypes.data_as(P(ctypes.c_float)))
        assert np.array_equal(codes, Q.pack(c_np, bits))
        assert np.array_equal(s.view(np.uint32), s_np.view(np.uint32))
        assert np.array_equal(b.view(np.uint32), b_np.view(np.uint32))
