"""The range exponent (include/kvq.h, kvq_qtensor.range_exp) on the CPU: the oracle's rule pinned by
its defining inequality at the boundaries, and the host-side computation the drop-in path uses for
triples that carry no registered word (kernels.range_exponent, which runs on any device) against
it. The GPU appends' value of the word is checked in tests/test_gpu_range.py."""

import numpy as np
import pytest
import torch

from myinfer_amd import kernels
from oracle import quantize as Q


def _bits(x, dtype):
    return Q.to_bits(np.asarray(x, np.float32), dtype)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_oracle_rule_at_the_boundaries(dtype):
    z = _bits([0.0], dtype)
    # |b| alone: 32768 needs no scaling, the next value up needs 2^1; 65536 needs 2^1, above it 2^2
    assert Q.range_exponent(z, _bits([32768.0], dtype), dtype, 8) == 0
    assert Q.range_exponent(z, _bits([-32768.0], dtype), dtype, 8) == 0
    if dtype == "bfloat16":  # bf16 values above the fp16 range
        assert Q.range_exponent(z, _bits([33024.0], dtype), dtype, 8) == 1   # the next bf16 above 2^15
        assert Q.range_exponent(z, _bits([65536.0], dtype), dtype, 8) == 1
        assert Q.range_exponent(z, _bits([66048.0], dtype), dtype, 8) == 2
        assert Q.range_exponent(z, _bits([1.0e6], dtype), dtype, 8) == 5    # 2^15 * 2^5 = 1048576
        assert Q.range_exponent(z, _bits([3.0e38], dtype), dtype, 8) == 113  # 2^15 * 2^112 < 3.0e38 <= 2^128
        assert Q.range_exponent(_bits([3.0e38], dtype), _bits([3.0e38], dtype), dtype, 8) == 127  # b + n s = inf
    # the other extreme b + n s: b = 0, s = 200 at 8 bits -> 51000 -> E = 1; at 4 bits 3000 -> 0
    assert Q.range_exponent(_bits([200.0], dtype), z, dtype, 8) == 1
    assert Q.range_exponent(_bits([200.0], dtype), z, dtype, 4) == 0
    # MLX's groups: b the larger-magnitude extreme and s of the other sign, so |b + n s| <= |b|
    assert Q.range_exponent(_bits([-100.0], dtype), _bits([20000.0], dtype), dtype, 8) == 0
    # the maximum over groups
    assert Q.range_exponent(_bits([1.0, 1.0], dtype), _bits([0.0, 40000.0], dtype), dtype, 8) == 1


def test_oracle_rule_is_the_smallest_exponent():
    rng = np.random.default_rng(5)
    for _ in range(200):
        s = (rng.standard_normal(16) * 10.0 ** rng.uniform(0, 6)).astype(np.float32)
        b = (rng.standard_normal(16) * 10.0 ** rng.uniform(0, 7)).astype(np.float32)
        sb, bb = _bits(s, "bfloat16"), _bits(b, "bfloat16")
        e = Q.range_exponent(sb, bb, "bfloat16", 8)
        s32, b32 = Q.from_bits(sb, "bfloat16"), Q.from_bits(bb, "bfloat16")
        bound = np.maximum(np.abs(b32), np.abs(b32 + np.float32(255) * s32)).max()
        assert bound <= 32768.0 * 2.0**e
        assert e == 0 or bound > 32768.0 * 2.0 ** (e - 1)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_host_computation_matches_oracle(bits, dtype):
    rng = np.random.default_rng(11 + bits)
    for mag in (1.0, 1e3, 3e4, 1e5, 1e9):
        s = torch.from_numpy(rng.standard_normal((2, 3, 17, 2)).astype(np.float32) * mag / 100).to(dtype)
        b = torch.from_numpy(rng.standard_normal((2, 3, 17, 2)).astype(np.float32) * mag).to(dtype)
        if dtype == torch.float16 and not (torch.isfinite(s).all() and torch.isfinite(b).all()):
            continue
        codes = torch.zeros((2, 3, 17, 128 * bits // 32), dtype=torch.int32)
        got = kernels.range_exponent((codes, s, b), bits)
        nd = "float16" if dtype == torch.float16 else "bfloat16"
        want = Q.range_exponent(s.view(torch.int16).numpy().view(np.uint16),
                                b.view(torch.int16).numpy().view(np.uint16), nd, bits)
        assert got.dtype == torch.int32 and got.shape == (1,)
        assert int(got) == want, (mag, int(got), want)


def test_host_computation_ignores_nan_groups_and_handles_empty():
    s = torch.tensor([[[[1.0], [float("nan")]]]], dtype=torch.bfloat16)
    b = torch.tensor([[[[40000.0], [float("nan")]]]], dtype=torch.bfloat16)
    codes = torch.zeros((1, 1, 2, 32), dtype=torch.int32)
    assert int(kernels.range_exponent((codes, s, b), 8)) == 1
    e = kernels.range_exponent((codes[:, :, :0], s[:, :, :0], b[:, :, :0]), 8)
    assert int(e) == 0


def test_registry_follows_views_and_drops_dead_buffers():
    codes = torch.zeros((1, 2, 512, 32), dtype=torch.int32).view(torch.uint32)
    word = torch.zeros(1, dtype=torch.int32)
    kernels.register_range_word(codes, word)
    assert kernels.range_word(codes[:, :, :100]) is word
    assert kernels.range_word(torch.zeros_like(codes)) is None
    with pytest.raises(ValueError):
        kernels.register_range_word(codes, torch.zeros(2, dtype=torch.int32))
    del codes
    other = torch.zeros((1, 2, 512, 32), dtype=torch.int32)
    assert kernels.range_word(other) is None or kernels.range_word(other) is not word
