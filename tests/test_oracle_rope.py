"""Pins the CPU restatement of RoPE (oracle/rope.py).

Checks chosen so that a plausible slip fails one of them: a wrong sign in either output of a pair
(unit-vector known answers, norm preservation), the wrong pair layout (NeoX halves vs interleaved
known answers), a wrong frequency exponent (hand-computed frequencies), positions not multiplied
by `scale` or not offset by `offset` (exact position identities), an angle that is not linear in
the position (composition of rotations), and dims past `dims` touched. An independent complex-
number formulation in float64 (torch) bounds the whole result.
"""

import math

import numpy as np
import pytest
import torch

from oracle import quantize as OQ
from oracle import rope as OR

F32 = np.float32


def _unit(D, i, L=1):
    x = np.zeros((L, D), F32)
    x[:, i] = 1.0
    return x


def test_frequencies_by_hand():
    f = OR.freqs(8, 10000.0)
    np.testing.assert_array_equal(f, np.array([1.0, 0.1, 0.01, 0.001], F32))
    f = OR.freqs(4, 100.0)
    np.testing.assert_array_equal(f, np.array([1.0, 0.1], F32))
    assert OR.freqs(128, 500000.0)[0] == 1.0


@pytest.mark.parametrize("traditional", [False, True])
def test_position_zero_is_identity(traditional):
    x = np.random.default_rng(0).standard_normal((3, 1, 64)).astype(F32)
    np.testing.assert_array_equal(OR.rope_f32(x, 64, traditional, 10000.0, 1.0, 0), x)


def test_neox_unit_vectors():
    D, dims, p = 16, 8, 3
    # pair i of the split-half layout is (i, i + dims/2), angle p * 10000^(-2i/dims)
    for i in range(dims // 2):
        th = p * 10000.0 ** (-2 * i / dims)
        y = OR.rope_f32(_unit(D, i), dims, False, 10000.0, 1.0, p)[0]
        want = np.zeros(D)
        want[i], want[i + dims // 2] = math.cos(th), math.sin(th)
        np.testing.assert_allclose(y, want, atol=2e-6)
        y = OR.rope_f32(_unit(D, i + dims // 2), dims, False, 10000.0, 1.0, p)[0]
        want = np.zeros(D)
        want[i], want[i + dims // 2] = -math.sin(th), math.cos(th)
        np.testing.assert_allclose(y, want, atol=2e-6)


def test_interleaved_unit_vectors():
    D, dims, p = 16, 8, 5
    for i in range(dims // 2):
        th = p * 10000.0 ** (-2 * i / dims)
        y = OR.rope_f32(_unit(D, 2 * i), dims, True, 10000.0, 1.0, p)[0]
        want = np.zeros(D)
        want[2 * i], want[2 * i + 1] = math.cos(th), math.sin(th)
        np.testing.assert_allclose(y, want, atol=2e-6)
        y = OR.rope_f32(_unit(D, 2 * i + 1), dims, True, 10000.0, 1.0, p)[0]
        want = np.zeros(D)
        want[2 * i], want[2 * i + 1] = -math.sin(th), math.cos(th)
        np.testing.assert_allclose(y, want, atol=2e-6)


@pytest.mark.parametrize("traditional", [False, True])
def test_norm_preserved_and_tail_untouched(traditional):
    D, dims = 128, 64
    x = np.random.default_rng(1).standard_normal((2, 40, D)).astype(F32)
    y = OR.rope_f32(x, dims, traditional, 10000.0, 1.0, 1000)
    np.testing.assert_array_equal(y[..., dims:], x[..., dims:])
    if traditional:
        nx = x[..., 0:dims:2] ** 2 + x[..., 1:dims:2] ** 2
        ny = y[..., 0:dims:2] ** 2 + y[..., 1:dims:2] ** 2
    else:
        nx = x[..., : dims // 2] ** 2 + x[..., dims // 2: dims] ** 2
        ny = y[..., : dims // 2] ** 2 + y[..., dims // 2: dims] ** 2
    np.testing.assert_allclose(ny, nx, rtol=2e-6, atol=1e-6)


@pytest.mark.parametrize("traditional", [False, True])
def test_offset_and_scale_are_positions(traditional):
    x = np.random.default_rng(2).standard_normal((1, 6, 64)).astype(F32)
    full = OR.rope_f32(np.repeat(x[:, :1], 20, axis=1), 64, traditional, 10000.0, 1.0, 0)
    # row l of a call at offset o sits at position o + l
    one = OR.rope_f32(x[:, :1], 64, traditional, 10000.0, 1.0, 13)
    np.testing.assert_array_equal(one[0, 0], full[0, 13])
    # scale multiplies the position: scale 0.5 at position 2p is position p, exactly
    for p in (1, 7, 9):
        a = OR.rope_f32(x[:, :1], 64, traditional, 10000.0, 0.5, 2 * p)
        b = OR.rope_f32(x[:, :1], 64, traditional, 10000.0, 1.0, p)
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("traditional", [False, True])
def test_rotations_compose(traditional):
    x = np.random.default_rng(3).standard_normal((4, 1, 64)).astype(F32)
    a = OR.rope_f32(OR.rope_f32(x, 64, traditional, 10000.0, 1.0, 17), 64, traditional, 10000.0, 1.0, 25)
    b = OR.rope_f32(x, 64, traditional, 10000.0, 1.0, 42)
    np.testing.assert_allclose(a, b, atol=2e-5)


def _complex_rope(x: torch.Tensor, dims, traditional, base, scale, offset):
    """float64 RoPE as multiplication of complex pairs by exp(i * theta)."""
    L = x.shape[-2]
    pos = (offset + torch.arange(L, dtype=torch.float64)) * scale
    inv = base ** (-torch.arange(0, dims, 2, dtype=torch.float64) / dims)
    rot = torch.polar(torch.ones(L, dims // 2, dtype=torch.float64), pos[:, None] * inv[None, :])
    out = x.clone()
    if traditional:
        z = torch.view_as_complex(x[..., :dims].reshape(*x.shape[:-1], dims // 2, 2).contiguous())
        out[..., :dims] = torch.view_as_real(z * rot).reshape(*x.shape[:-1], dims)
    else:
        z = torch.complex(x[..., : dims // 2], x[..., dims // 2: dims]) * rot
        out[..., : dims // 2], out[..., dims // 2: dims] = z.real, z.imag
    return out


@pytest.mark.parametrize("traditional", [False, True])
@pytest.mark.parametrize("dims,base,scale,offset", [(128, 10000.0, 1.0, 0), (64, 500000.0, 0.25, 4096),
                                                     (128, 1000000.0, 1.0, 30000)])
def test_against_complex_float64(traditional, dims, base, scale, offset):
    x = np.random.default_rng(4).standard_normal((2, 3, 33, 128)).astype(F32)
    y = OR.rope_f32(x, dims, traditional, base, scale, offset)
    ref = _complex_rope(torch.from_numpy(x).double(), dims, traditional, base, scale, offset).numpy()
    # the fp32 angle carries a relative error of ~1e-7, so the bound grows with the position
    atol = 4e-6 + 2e-7 * (offset + 33) * scale * float(np.abs(x).max())
    np.testing.assert_allclose(y, ref, atol=atol)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_rounded_and_quantized(dtype):
    x = np.random.default_rng(5).standard_normal((1, 2, 9, 128)).astype(F32)
    xb = OQ.to_bits(x, dtype)
    yb = OR.rope(xb, dtype, 128, False, 10000.0, 1.0, 77)
    np.testing.assert_array_equal(yb, OQ.to_bits(OR.rope_f32(OQ.from_bits(xb, dtype), 128, False, 10000.0, 1.0, 77),
                                                 dtype))
    c, s, b = OR.rope_quantize(xb, dtype, 64, 8, 128, False, 10000.0, 1.0, 77)
    c2, s2, b2 = OQ.quantize(yb, dtype, 64, 8)
    assert np.array_equal(c, c2) and np.array_equal(s, s2) and np.array_equal(b, b2)
