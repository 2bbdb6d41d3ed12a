"""kernels.fits_fp16_operands on the CPU: whether a quantized cache's dequantized values fit the fp16
range that the prefill kernel's operands need (a bf16 cache beyond it makes prefill return NaN rows;
see tests/test_gpu_range.py). The triples come from the oracle quantizer, so the check sees the
same scales and biases the append kernel writes (bit-exact with it)."""

import numpy as np
import pytest
import torch

from myinfer_amd import kernels
from oracle import quantize as OQ


def bf16_triple(x: np.ndarray, bits: int, group: int = 64):
    xb = torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16)
    codes, scales, biases = OQ.quantize(xb.view(torch.int16).numpy().view(np.uint16), "bfloat16", group, bits)
    as_bf16 = lambda a: torch.from_numpy(a.astype(np.uint16).view(np.int16)).view(torch.bfloat16)
    return torch.from_numpy(codes.astype(np.int64)), as_bf16(scales), as_bf16(biases)


@pytest.mark.parametrize("bits", [8, 4])
def test_normal_cache_fits(bits):
    x = np.random.default_rng(1).standard_normal((2, 4, 33, 128)) * 3.0
    assert kernels.fits_fp16_operands(bf16_triple(x, bits), bits)


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("big", [7e4, -7e4, 2e6])
def test_group_beyond_fp16_range_is_flagged(bits, big):
    x = np.random.default_rng(2).standard_normal((1, 2, 40, 128))
    x[0, 1, 17, 70] = big  # one element of one group of one row
    assert not kernels.fits_fp16_operands(bf16_triple(x, bits), bits)
    x[0, 1, 17, 70] = 6e4  # just inside
    assert kernels.fits_fp16_operands(bf16_triple(x, bits), bits)


def test_either_extreme_of_a_group_counts():
    # a hand-made triple whose bias fits but whose largest code overshoots: 60000 + 255 * 100
    s = torch.full((1, 1, 2, 2), 0.01, dtype=torch.bfloat16)
    b = torch.zeros_like(s)
    codes = torch.zeros((1, 1, 2, 32), dtype=torch.int64)
    assert kernels.fits_fp16_operands((codes, s, b), 8)
    s[0, 0, 1, 1], b[0, 0, 1, 1] = 100.0, 60000.0
    assert not kernels.fits_fp16_operands((codes, s, b), 8)
    assert kernels.fits_fp16_operands((codes, s, b), 2)  # 60000 + 3 * 100 fits
    b[0, 0, 0, 0] = float("inf")
    assert not kernels.fits_fp16_operands((codes, s, b), 2)
