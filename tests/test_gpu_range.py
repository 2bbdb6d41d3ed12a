"""bf16 caches whose values leave the fp16 range.

MLX stores a bf16 cache's scales and biases in bf16, so a group may hold values beyond 65504. The
prefill kernels' dequantized operands are fp16 (head_dim 64/128 and head_dim 256 alike): a row
block that reads such a group returns NaN (not finite wrong values), and every other row block
stays exact. The decode kernel applies key
scales and biases in fp32 and takes |x| up to about 1.3e5 in values (the probability times value
scale is an fp16 operand), so it stays exact for the same cache.
"""

import math

import numpy as np
import pytest
import torch

from myinfer_amd import kernels
from tests.helpers import assert_close, exact_reference, seeded_normal

pytestmark = pytest.mark.gpu
DEV = "cuda"


def big_cache(B, Hkv, S, D, bits, big_head, kmul, vmul, seed):
    k = seeded_normal((B, Hkv, S, D), seed, torch.float32)
    v = seeded_normal((B, Hkv, S, D), seed + 1, torch.float32)
    k[:, big_head] *= kmul
    v[:, big_head] *= vmul
    trip = []
    for x in (k.to(torch.bfloat16).to(DEV), v.to(torch.bfloat16).to(DEV)):
        codes = torch.zeros((B, Hkv, S, D * bits // 32), dtype=torch.int32, device=DEV).view(torch.uint32)
        sc = torch.zeros((B, Hkv, S, D // 64), dtype=torch.bfloat16, device=DEV)
        bi = torch.zeros_like(sc)
        kernels.quantize_append(x, (codes, sc, bi), row_offset=0, group_size=64, bits=bits)
        trip.append((codes, sc, bi))
    return trip[0], trip[1]


@pytest.mark.parametrize("which", ["keys", "values"])
@pytest.mark.parametrize("causal", [False, True])
def test_prefill_poisons_row_blocks_beyond_fp16(which, causal):
    print(f"range prefill which={which} causal={causal}", flush=True)
    B, Hq, Hkv, L, S, D, bits = 1, 8, 2, 64, 700, 128, 8
    kmul, vmul = (4e4, 1.0) if which == "keys" else (1.0, 4e4)  # about 1.6e5 at the extremes
    kt, vt = big_cache(B, Hkv, S, D, bits, 1, kmul, vmul, 300)
    assert float((kt[2] if which == "keys" else vt[2])[:, 1].float().abs().max()) > 65504
    # the host-side check flags exactly the cache that prefill cannot hold
    assert not kernels.fits_fp16_operands(kt if which == "keys" else vt, bits)
    assert kernels.fits_fp16_operands(vt if which == "keys" else kt, bits)
    assert kernels.fits_fp16_operands(tuple(t[:, :1] for t in kt), bits)
    q = seeded_normal((B, Hq, L, D), 302, torch.bfloat16, DEV)
    scale = 1.0 / math.sqrt(D)
    out = kernels.attention(q, kt, vt, scale, causal=causal, bits=bits, kernel="prefill")
    torch.cuda.synchronize()
    o = out.cpu().float()
    # KV head 1 (query heads 4..7) reads the out-of-range groups: every row is NaN
    assert torch.isnan(o[:, 4:]).all()
    # KV head 0 is untouched and exact
    ref = exact_reference(q[:, :4], tuple(t[:, :1] for t in kt), tuple(t[:, :1] for t in vt), scale, bits=bits,
                          causal=causal)
    assert_close(out[:, :4], ref, "in-range head")


def test_decode_exact_beyond_fp16():
    print("range decode", flush=True)
    B, Hq, Hkv, L, S, D, bits = 1, 16, 2, 1, 900, 128, 8
    # keys up to about 1.6e5 (folded in fp32), values up to about 8e4 (value scale about 600)
    kt, vt = big_cache(B, Hkv, S, D, bits, 1, 4e4, 2e4, 310)
    q = (0.01 * seeded_normal((B, Hq, L, D), 312, torch.float32)).to(torch.bfloat16).to(DEV)
    scale = 1.0 / math.sqrt(D)
    out = kernels.attention(q, kt, vt, scale, bits=bits, kernel="decode")
    torch.cuda.synchronize()
    ref = exact_reference(q, kt, vt, scale, bits=bits)
    assert np.isfinite(out.cpu().float().numpy()).all()
    assert_close(out, ref, "decode beyond fp16")


@pytest.mark.parametrize("which", ["keys", "values"])
@pytest.mark.parametrize("L,S,causal", [(64, 700, True), (200, 900, False), (16, 12000, True)])
def test_head_dim_256_poisons_beyond_fp16(which, L, S, causal):
    # wide_attn_kernel (head_dim 256) dequantizes to fp16 operands as well; (16, 12000) splits the
    # key range over workgroups, so the poisoned partials must reach the output through the merge
    print(f"range wide which={which} L={L} S={S} causal={causal}", flush=True)
    B, Hq, Hkv, D, bits = 1, 8, 2, 256, 8
    kmul, vmul = (4e4, 1.0) if which == "keys" else (1.0, 4e4)
    kt, vt = big_cache(B, Hkv, S, D, bits, 1, kmul, vmul, 320 + L)
    assert not kernels.fits_fp16_operands(kt if which == "keys" else vt, bits)
    q = seeded_normal((B, Hq, L, D), 322 + L, torch.bfloat16, DEV)
    scale = 1.0 / math.sqrt(D)
    out = kernels.attention(q, kt, vt, scale, causal=causal, bits=bits, kernel="prefill")
    torch.cuda.synchronize()
    o = out.cpu().float()
    assert torch.isnan(o[:, 4:]).all()
    ref = exact_reference(q[:, :4], tuple(t[:, :1] for t in kt), tuple(t[:, :1] for t in vt), scale, bits=bits,
                          causal=causal)
    assert_close(out[:, :4], ref, "wide in-range head")
