"""GPU RoPE: the in-place query rotation (kvq_rope) against the CPU restatement, and the fused
rotate-and-quantize append (kvq_rope_quantize_append) against quantizing the rotated keys.

Tolerance of the rotation: the GPU takes sin/cos of the fp32 angle with the device's fp32
sincosf (within about 1 fp32 ulp), the restatement takes the correctly rounded values, so a
rotated element may round to a neighbouring value of its dtype. Each element must lie within one
ulp of its dtype (plus 2^-22 of the row's largest input, for cancellation in a*cos - b*sin) and at
most 0.2% of the elements may differ at all. The fused append must store exactly what quantizing
the GPU's own rotated keys stores (codes, scales and biases bit-identical), so the fused path is
pinned to the restatement through the same bound."""

import numpy as np
import pytest
import torch

from myinfer_amd import kernels
from myinfer_amd.cache import QuantizedKVCache
from oracle import quantize as OQ
from oracle import rope as OR
from tests.helpers import NP_DTYPE, seeded_normal, to_np_bits

pytestmark = pytest.mark.gpu
DEV = "cuda"
MANT = {torch.float16: 10, torch.bfloat16: 7}


def _alloc(B, H, cap, D, bits, G, dtype):
    codes = torch.zeros((B, H, cap, D * bits // 32), dtype=torch.int32, device=DEV).view(torch.uint32)
    scales = torch.zeros((B, H, cap, D // G), dtype=dtype, device=DEV)
    return codes, scales, torch.zeros_like(scales)


def _assert_rope_close(got: torch.Tensor, x: torch.Tensor, r: kernels.Rope, offset: int, what: str):
    dt = NP_DTYPE[x.dtype]
    ref_bits = OR.rope(to_np_bits(x), dt, r.dims, r.traditional, r.base, r.scale, offset)
    got_bits = to_np_bits(got)
    D = x.shape[-1]
    # dims past r.dims pass through untouched
    assert np.array_equal(got_bits[..., r.dims:], to_np_bits(x)[..., r.dims:]), f"{what}: tail modified"
    ref = OQ.from_bits(ref_bits, dt).astype(np.float64)
    g = OQ.from_bits(got_bits, dt).astype(np.float64)
    assert np.isfinite(g).all(), f"{what}: non-finite"
    mag = np.maximum(np.abs(ref), np.abs(g))
    ulp = np.exp2(np.floor(np.log2(np.maximum(mag, 1e-30))) - MANT[x.dtype])
    rowmax = np.abs(x.float().cpu().numpy()).max(axis=-1, keepdims=True).astype(np.float64)
    bound = ulp + 2.0**-22 * rowmax
    err = np.abs(g - ref)
    assert (err <= bound).all(), f"{what}: max err {err.max()} at {np.unravel_index(np.argmax(err - bound), err.shape)}"
    frac = float((got_bits != ref_bits).mean())
    assert frac <= 2e-3, f"{what}: {frac:.2e} of the elements differ from the restatement (D={D})"
    return frac


CASES = [
    # (dims, traditional, base, scale, offset)
    (128, False, 10000.0, 1.0, 0),
    (128, True, 10000.0, 1.0, 0),
    (64, False, 500000.0, 1.0, 4093),
    (64, True, 1000000.0, 0.25, 31000),
    (128, False, 1000000.0, 1.0, 32760),
    (16, False, 10000.0, 1.0, 7),
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("case", CASES)
def test_rope_in_place_vs_oracle(dtype, case):
    dims, trad, base, scale, offset = case
    print(f"rope dtype={dtype} dims={dims} traditional={trad} base={base} scale={scale} offset={offset}", flush=True)
    r = kernels.Rope(dims, trad, base, scale)
    x = seeded_normal((2, 5, 37, 128), 7 + dims, dtype)
    x[0, 1, 3] *= 30.0
    y = x.to(DEV)
    assert kernels.rope(y, r, offset) is y
    torch.cuda.synchronize()
    _assert_rope_close(y, x, r, offset, "rope")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_rope_strided_head_dim_64(dtype):
    # a [B, L, H, D] projection viewed as [B, H, L, D]: strided rows, head_dim 64
    print(f"rope strided D=64 dtype={dtype}", flush=True)
    r = kernels.Rope(64, False, 10000.0, 1.0)
    base = seeded_normal((3, 19, 4, 64), 21, dtype).to(DEV)
    view = base.transpose(1, 2)
    x = view.cpu().clone()
    kernels.rope(view, r, 100)
    torch.cuda.synchronize()
    _assert_rope_close(view, x, r, 100, "rope strided")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits,G", [(8, 64), (4, 64), (4, 32), (2, 128)])
@pytest.mark.parametrize("trad", [False, True])
def test_fused_append_equals_quantized_rotation(dtype, bits, G, trad):
    print(f"rope_quantize_append dtype={dtype} bits={bits} G={G} traditional={trad}", flush=True)
    B, H, L, D, row_offset, pos = 2, 3, 45, 128, 9, 2000
    r = kernels.Rope(128 if G != 32 else 64, trad, 10000.0, 1.0)
    k = seeded_normal((B, H, L, D), 31 + bits, dtype).to(DEV)
    v = seeded_normal((B, H, L, D), 41 + bits, dtype).to(DEV)
    k_keep = k.clone()
    kd, vd = _alloc(B, H, 64, D, bits, G, dtype), _alloc(B, H, 64, D, bits, G, dtype)
    kernels.quantize_append(k, kd, v, vd, row_offset=row_offset, group_size=G, bits=bits, rope=r, rope_offset=pos)
    kr = kernels.rope(k.clone(), r, pos)
    torch.cuda.synchronize()
    assert torch.equal(k, k_keep), "the fused append modified its source keys"
    _assert_rope_close(kr, k_keep.cpu(), r, pos, "rotated keys")
    dt = NP_DTYPE[dtype]
    sl = slice(row_offset, row_offset + L)
    for src, dst, what in ((kr, kd, "K"), (v, vd, "V")):
        ref_c, ref_s, ref_b = OQ.quantize(to_np_bits(src), dt, G, bits)
        got_c = dst[0][:, :, sl].cpu().view(torch.int32).numpy().view(np.uint32)
        assert np.array_equal(got_c, ref_c), f"{what} codes differ"
        assert np.array_equal(to_np_bits(dst[1][:, :, sl]), ref_s), f"{what} scales differ"
        assert np.array_equal(to_np_bits(dst[2][:, :, sl]), ref_b), f"{what} biases differ"
    # rows outside the written range are untouched
    assert int(kd[0][:, :, :row_offset].view(torch.int32).abs().sum()) == 0
    assert int(kd[0][:, :, row_offset + L:].view(torch.int32).abs().sum()) == 0
    # against the restatement end to end: groups that saw no rounding flip are bit-identical
    oc, os_, ob = OR.rope_quantize(to_np_bits(k_keep), dt, G, bits, r.dims, trad, 10000.0, 1.0, pos)
    same = (to_np_bits(kd[1][:, :, sl]) == os_) & (to_np_bits(kd[2][:, :, sl]) == ob)
    assert same.mean() >= 0.95, f"only {same.mean():.3f} of the K groups match the restatement"


def test_fused_append_prefill_chunk_shape():
    # a 2048-row bf16 prefill chunk of the long-context configuration, keys at positions 14336..
    print("rope_quantize_append bf16 [1, 8, 2048, 128] offset 14336", flush=True)
    r = kernels.Rope(128, False, 1000000.0, 1.0)
    k = seeded_normal((1, 8, 2048, 128), 5, torch.bfloat16).to(DEV)
    v = seeded_normal((1, 8, 2048, 128), 6, torch.bfloat16).to(DEV)
    kd, vd = _alloc(1, 8, 16384, 128, 8, 64, torch.bfloat16), _alloc(1, 8, 16384, 128, 8, 64, torch.bfloat16)
    kernels.quantize_append(k, kd, v, vd, row_offset=14336, group_size=64, bits=8, rope=r)
    kr = kernels.rope(k.clone(), r, 14336)
    torch.cuda.synchronize()
    _assert_rope_close(kr, k.cpu(), r, 14336, "rotated keys")
    ref = kernels.quantize(kr, group_size=64, bits=8)
    for got, want in zip(kd, ref):
        assert torch.equal(got[:, :, 14336:], want)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_cache_appends_in_pieces_match_one_append(dtype):
    # keys appended in pieces are rotated at their absolute positions: the same cache as one call
    print(f"cache rope pieces dtype={dtype}", flush=True)
    r = kernels.Rope(128, False, 10000.0, 1.0)
    B, H, D = 1, 4, 128
    k = seeded_normal((B, H, 300, D), 51, dtype).to(DEV)
    v = seeded_normal((B, H, 300, D), 52, dtype).to(DEV)
    a = QuantizedKVCache(group_size=64, bits=8)
    for lo, hi in ((0, 100), (100, 101), (101, 256), (256, 300)):
        a.update_and_fetch(k[:, :, lo:hi].contiguous(), v[:, :, lo:hi].contiguous(), rope=r)
    b = QuantizedKVCache(group_size=64, bits=8)
    b.update_and_fetch(k, v, rope=r)
    torch.cuda.synchronize()
    assert a.offset == b.offset == 300
    for x, y in zip((*a.keys, *a.values), (*b.keys, *b.values)):
        assert torch.equal(x[:, :, :300], y[:, :, :300])


def test_rope_then_attention_depends_on_relative_position():
    # q at position m and k at position n rotated by the GPU: q.k depends only on m - n
    print("rope relative position", flush=True)
    r = kernels.Rope(128, False, 10000.0, 1.0)
    q = seeded_normal((1, 1, 1, 128), 61, torch.float16)
    k = seeded_normal((1, 1, 1, 128), 62, torch.float16)
    dots = []
    for m, n in ((5, 0), (105, 100), (4005, 4000)):
        qr = kernels.rope(q.to(DEV), r, m).float()
        kr = kernels.rope(k.to(DEV), r, n).float()
        dots.append(float((qr * kr).sum()))
    # fp16 rounding of the rotated rows and the fp32 angle (error ~ position * 2^-24 rad) bound the
    # spread; a rotation that is not a function of m - n moves the dot by O(|q| |k|)
    assert max(dots) - min(dots) <= 1e-2 * float(q.float().norm() * k.float().norm()), dots


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("use_rope", [False, True])
@pytest.mark.parametrize("with_v", [False, True])
def test_prepared_append_equals_append(dtype, use_rope, with_v):
    # prepare_append builds the descriptors once; each call must store exactly what quantize_append
    # stores, for strided sources and successive offsets
    print(f"prepared append dtype={dtype} rope={use_rope} v={with_v}", flush=True)
    r = kernels.Rope(128, False, 10000.0, 1.0) if use_rope else None
    B, H, D, cap = 2, 4, 128, 320
    src_k = seeded_normal((B, 300, H, D), 71, dtype).to(DEV).transpose(1, 2)  # [B, H, L, D], strided
    src_v = seeded_normal((B, H, 300, D), 72, dtype).to(DEV)
    a_k, a_v = _alloc(B, H, cap, D, 4, 64, dtype), _alloc(B, H, cap, D, 4, 64, dtype)
    b_k, b_v = _alloc(B, H, cap, D, 4, 64, dtype), _alloc(B, H, cap, D, 4, 64, dtype)
    call = kernels.prepare_append(b_k, b_v if with_v else None, group_size=64, bits=4, rope=r)
    for lo, hi in ((0, 1), (1, 130), (130, 131), (131, 300)):
        k, v = src_k[:, :, lo:hi], src_v[:, :, lo:hi] if with_v else None
        kernels.quantize_append(k, a_k, v, a_v if with_v else None, row_offset=lo + 7, group_size=64, bits=4,
                                rope=r, rope_offset=lo + 100)
        call(k, v, lo + 7, rope_offset=lo + 100)
    torch.cuda.synchronize()
    for x, y in zip((*a_k, *a_v), (*b_k, *b_v)):
        assert torch.equal(x, y)
    with pytest.raises(ValueError):
        call(src_k[:, :, :20], None, cap - 19)  # past the last row
    with pytest.raises(ValueError):
        call(src_k[:1, :, :4], None, 0)  # batch does not match the destination
    with pytest.raises(ValueError):
        call(src_k[:, :, :4].float(), None, 0)  # dtype differs
