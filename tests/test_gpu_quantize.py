"""GPU quantize-and-append kernel: codes, scales and biases bit-identical to the CPU restatement
of MLX's affine quantizer, for every supported (dtype, bits, group) and at the BASELINE shapes."""

import numpy as np
import pytest
import torch

from myinfer_amd import kernels
from oracle import quantize as OQ
from tests.helpers import NP_DTYPE, seeded_normal, to_np_bits

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _alloc(B, H, cap, D, bits, G, dtype):
    codes = torch.zeros((B, H, cap, D * bits // 32), dtype=torch.int32, device=DEV).view(torch.uint32)
    scales = torch.zeros((B, H, cap, D // G), dtype=dtype, device=DEV)
    return codes, scales, torch.zeros_like(scales)


def _check_rows(x: torch.Tensor, dst, row_offset, bits, G):
    dt = NP_DTYPE[x.dtype]
    L = x.shape[2]
    ref_c, ref_s, ref_b = OQ.quantize(to_np_bits(x), dt, G, bits)
    codes, scales, biases = dst
    got_c = codes[:, :, row_offset:row_offset + L].cpu().view(torch.int32).numpy().view(np.uint32)
    assert np.array_equal(got_c, ref_c), "codes differ"
    assert np.array_equal(to_np_bits(scales[:, :, row_offset:row_offset + L]), ref_s), "scales differ"
    assert np.array_equal(to_np_bits(biases[:, :, row_offset:row_offset + L]), ref_b), "biases differ"


def _stress(shape, seed, dtype):
    x = seeded_normal(shape, seed, torch.float32)
    x[..., ::7, :] *= 8.0
    x[..., 3::11, 5] = 40.0
    x[..., 5::13, :] = x[..., 5::13, :].abs()
    x[..., 6::13, :] = -x[..., 6::13, :].abs()
    x[..., 9::17, :] = 0.0
    x[..., 10::17, :] = 0.75
    return x.to(dtype).to(DEV)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("G", [32, 64, 128])
def test_bit_exact_vs_oracle(dtype, bits, G):
    print(f"quantize dtype={dtype} bits={bits} G={G}", flush=True)
    B, H, L, D = 2, 3, 37, 128
    x = _stress((B, H, L, D), 11 + bits + G, dtype)
    dst = _alloc(B, H, 64, D, bits, G, dtype)
    kernels.quantize_append(x, dst, row_offset=5, group_size=G, bits=bits)
    _check_rows(x, dst, 5, bits, G)
    # rows outside the written range are untouched
    assert int(dst[0][:, :, :5].view(torch.int32).abs().sum()) == 0
    assert int(dst[0][:, :, 5 + L:].view(torch.int32).abs().sum()) == 0


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_known_answer_groups(dtype):
    D = 128
    rows = torch.zeros((4, D), dtype=torch.float32)
    rows[1] = 0.5
    rows[2, :64] = torch.arange(64.0)
    rows[2, 64:] = -torch.arange(64.0)
    rows[3] = torch.linspace(-3, 5, D)
    x = rows.to(dtype).to(DEV).reshape(1, 1, 4, D)
    dst = _alloc(1, 1, 4, D, 8, 64, dtype)
    kernels.quantize_append(x, dst, group_size=64, bits=8)
    _check_rows(x, dst, 0, 8, 64)
    c = dst[0].cpu().view(torch.int32).numpy().view(np.uint32)[0, 0]
    codes = OQ.unpack(c, 8)
    assert (codes[0] == 0).all() and (codes[1] == 0).all()
    assert codes[2, 0] == 255 and codes[2, 63] == 0 and codes[2, 64] == 255 and codes[2, 127] == 0
    if dtype == torch.float16:
        assert int(to_np_bits(dst[1])[0, 0, 0, 0]) == 0x8002


def test_strided_sources_and_fused_kv():
    B, L, H, D = 2, 19, 4, 128
    dtype = torch.bfloat16
    kx = seeded_normal((B, L, H, D), 21, dtype, DEV).transpose(1, 2)  # [B, H, L, D] view, strided
    vx = seeded_normal((B, L, H, D), 22, dtype, DEV).transpose(1, 2)
    kd = _alloc(B, H, 256, D, 4, 64, dtype)
    vd = _alloc(B, H, 256, D, 4, 64, dtype)
    kernels.quantize_append(kx, kd, vx, vd, row_offset=100, group_size=64, bits=4)
    _check_rows(kx.contiguous(), kd, 100, 4, 64)
    _check_rows(vx.contiguous(), vd, 100, 4, 64)


@pytest.mark.parametrize("name,B,H,L,D,bits,dtype", [
    ("C1-append", 1, 8, 1, 128, 8, torch.float16),
    ("C1-bulk", 1, 8, 4096, 128, 8, torch.float16),
    ("C3-chunk", 1, 4, 512, 128, 8, torch.bfloat16),
    ("C4-4bit", 1, 8, 2048, 128, 4, torch.float16),
    ("C5-decode", 4, 16, 1, 128, 8, torch.bfloat16),
    ("D64", 1, 4, 700, 64, 8, torch.float16),
])
def test_baseline_shapes(name, B, H, L, D, bits, dtype):
    print(f"quantize shape case {name}", flush=True)
    x = _stress((B, H, L, D), 1000 + B * H + L, dtype)
    dst = _alloc(B, H, L + 3, D, bits, 64, dtype)
    kernels.quantize_append(x, dst, row_offset=3, group_size=64, bits=bits)
    _check_rows(x, dst, 3, bits, 64)


@pytest.mark.parametrize("D,G,bits", [(96, 32, 8), (192, 64, 4), (320, 64, 8), (384, 128, 2), (32, 32, 8)])
def test_row_widths_that_are_not_powers_of_two(D, G, bits):
    """mx.quantize takes any row width that is a multiple of the group size: rows of D / 32
    threads that do not divide a wave evenly, and a single-thread row."""
    print(f"quantize D={D} G={G} bits={bits}", flush=True)
    B, H, L = 2, 3, 45
    x = _stress((B, H, L, D), 500 + D, torch.bfloat16)
    dst = _alloc(B, H, L + 2, D, bits, G, torch.bfloat16)
    kernels.quantize_append(x, dst, row_offset=2, group_size=G, bits=bits)
    _check_rows(x, dst, 2, bits, G)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_half_integer_quotients(dtype):
    """Groups whose quotients (x - bias) / s are exact half-integers (ties, rounded half to even)
    and integers: a group spans [0, 255 * 2^-k], so s = -2^-k and bias = its maximum, and the other
    values sit on the 2^-(k+1) grid. The kernel's fast quotient must hand every tie to the exact
    division; the codes must equal the CPU restatement's."""
    print(f"quantize ties dtype={dtype}", flush=True)
    D, G = 128, 64
    rows = []
    for k in range(0, 6):
        for shift in range(2):
            top = 255.0 * 2.0 ** -k
            step = 2.0 ** -(k + 1)
            g = (torch.arange(G, dtype=torch.float64) * 2 + 1 + shift) % 510 * step  # odd multiples: ties
            g[0], g[1] = 0.0, top
            rows.append(torch.cat([g, g.flip(0)]))
    x = torch.stack(rows).to(torch.float32)
    assert torch.equal(x.to(dtype).to(torch.float32), x), "the grid values are exact in the dtype"
    x = x.to(dtype).to(DEV).reshape(1, 1, -1, D)
    dst = _alloc(1, 1, x.shape[2], D, 8, G, dtype)
    kernels.quantize_append(x, dst, group_size=G, bits=8)
    _check_rows(x, dst, 0, 8, G)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_c5_chunk_bit_exact(dtype):
    """A whole C5 prefill chunk (B = 4, 16 KV heads, 2048 rows, head_dim 128: 16.8M values per
    tensor) through the fused K/V launch: enough quotients land within a few ulp of a half-integer
    to exercise the exact-division path."""
    print(f"quantize C5 chunk dtype={dtype}", flush=True)
    B, H, L, D = 4, 16, 2048, 128
    kx = seeded_normal((B, H, L, D), 77, dtype, DEV)
    vx = seeded_normal((B, H, L, D), 78, dtype, DEV) * 3.0
    kd = _alloc(B, H, L + 16, D, 8, 64, dtype)
    vd = _alloc(B, H, L + 16, D, 8, 64, dtype)
    kernels.quantize_append(kx, kd, vx, vd, row_offset=16, group_size=64, bits=8)
    _check_rows(kx, kd, 16, 8, 64)
    _check_rows(vx, vd, 16, 8, 64)


def test_quantize_counterpart_of_mx_quantize():
    x = seeded_normal((3, 5, 256), 31, torch.float16, DEV)
    c, s, b = kernels.quantize(x, 64, 4)
    assert c.shape == (3, 5, 32) and s.shape == (3, 5, 4) and c.dtype == torch.uint32
    rc, rs, rb = OQ.quantize(to_np_bits(x), "float16", 64, 4)
    assert np.array_equal(c.cpu().view(torch.int32).numpy().view(np.uint32), rc)
    assert np.array_equal(to_np_bits(s), rs) and np.array_equal(to_np_bits(b), rb)
