"""bf16 caches whose values leave the fp16 range.

MLX stores a bf16 cache's scales and biases in bf16, so a group may hold values beyond 65504, and
the reference's MLX path computes them in bf16 (m5engine/attention.py:66-69, 87-90). The prefill
kernels here multiply fp16 operands: a cache keeps a range exponent E (include/kvq.h,
kvq_qtensor.range_exp) that its appends raise, and the prefill kernels stage the operands times
2^-E and fold 2^E back into the scores (K) and the output (V). Through the cache objects and the
drop-in entry points the results are finite and within the bars below; a raw prefill call whose
descriptors carry no range word keeps the old policy: the row blocks that read such a group return
NaN, never a finite wrong value. Decode applies scales and biases in fp32 and needs no scaling.

Bars: for values beyond the range, the bf16 bar (the fp16 V operands at 2^-E scale keep 11
significant bits). For keys beyond the range the scores are large (about 1e4 to 1e5 in natural-log
units) and the fp16 rounding of the keys moves them: the bar adds the error of exact fp64
attention whose dequantized keys carry the kernel's rounding (tests/test_gpu_range.staged_keys),
as the rising-key test does at fp16 scale.
"""

import math

import numpy as np
import pytest
import torch

from myinfer_amd import attention as A
from myinfer_amd import kernels
from myinfer_amd.cache import QuantizedKVCache
from myinfer_amd.paged import PagedRadixKVCache
from oracle import attention as OA
from oracle import quantize as OQ
from tests.helpers import TOL, assert_close, exact_reference, seeded_normal, to_np_bits, triple_to_np

pytestmark = pytest.mark.gpu
DEV = "cuda"


def big_rows(B, Hkv, S, D, big_head, kmul, vmul, seed):
    k = seeded_normal((B, Hkv, S, D), seed, torch.float32)
    v = seeded_normal((B, Hkv, S, D), seed + 1, torch.float32)
    k[:, big_head] *= kmul
    v[:, big_head] *= vmul
    return k.to(torch.bfloat16).to(DEV), v.to(torch.bfloat16).to(DEV)


def big_cache(B, Hkv, S, D, bits, big_head, kmul, vmul, seed):
    """Raw triples (no range word registered), as a foreign caller would build them."""
    trip = []
    for x in big_rows(B, Hkv, S, D, big_head, kmul, vmul, seed):
        codes = torch.zeros((B, Hkv, S, D * bits // 32), dtype=torch.int32, device=DEV).view(torch.uint32)
        sc = torch.zeros((B, Hkv, S, D // 64), dtype=torch.bfloat16, device=DEV)
        bi = torch.zeros_like(sc)
        kernels.quantize_append(x, (codes, sc, bi), row_offset=0, group_size=64, bits=bits)
        trip.append((codes, sc, bi))
    return trip[0], trip[1]


def oracle_range(tr, bits):
    _, s, b = tr
    return OQ.range_exponent(to_np_bits(s), to_np_bits(b), "bfloat16", bits)


def staged_keys(kt, bits, e):
    """The keys as the prefill kernels' K operands hold them, in the cache's units: scale and bias
    times 2^-e rounded to fp16, then one fp16 fused multiply-add per code (c s' + b'), times 2^e."""
    codes, sb, bb = triple_to_np(kt)
    c = OQ.unpack(codes, bits).astype(np.float64)
    s16 = (OQ.from_bits(sb, "bfloat16").astype(np.float64) * 2.0**-e).astype(np.float16).astype(np.float64)
    b16 = (OQ.from_bits(bb, "bfloat16").astype(np.float64) * 2.0**-e).astype(np.float16).astype(np.float64)
    D = c.shape[-1]
    cg = c.reshape(*c.shape[:-1], D // 64, 64)
    k16 = (cg * s16[..., None] + b16[..., None]).astype(np.float16).astype(np.float64)
    return k16.reshape(c.shape) * 2.0**e


def check_against_exact(out, q, kt, vt, scale, bits, ek, what, **mask):
    """Finite, and within the bf16 bar (plus the key-rounding floor of the kernel's scaled fp16 K
    operands when the keys needed scaling) against exact fp64 attention."""
    o = out.detach().cpu().float().numpy().astype(np.float64)
    assert np.isfinite(o).all(), f"{what}: non-finite output"
    ref = exact_reference(q, kt, vt, scale, bits=bits, **mask)
    max_abs, rel = TOL[torch.bfloat16](ref)
    st = OA.error_stats(o, ref)
    if ek > 0:
        kq = staged_keys(kt, bits, ek)
        vdq = OQ.dequantize(*triple_to_np(vt), "bfloat16", 64, bits)
        qn = q.detach().cpu().float().numpy().astype(np.float64)
        sl = mask.get("seq_lens")
        floor_ref = OA.exact_attention(qn, kq, vdq, scale, causal=mask.get("causal", False),
                                       window=mask.get("window", 0), seq_lens=sl)
        fl = OA.error_stats(floor_ref, ref)
        max_abs, rel = max_abs + fl["max_abs"], rel + fl["rel_l2"]
    assert st["max_abs"] <= max_abs and st["rel_l2"] <= rel, f"{what}: {st} vs bounds max_abs {max_abs}, rel_l2 {rel}"
    return st


@pytest.mark.parametrize("which", ["keys", "values"])
@pytest.mark.parametrize("D,L,S,causal", [(128, 64, 700, True), (128, 200, 900, False), (64, 64, 700, True),
                                          (256, 64, 700, True), (256, 16, 12000, True)])
def test_prefill_through_the_cache_is_finite(which, D, L, S, causal):
    """The drop-in path: a QuantizedKVCache appends bf16 rows of about 1.6e5 (its range word is
    raised as the oracle says) and blocked_quantized_sdpa's prefill over its views is finite and
    within the bars. (256, 16, 12000) splits the keys over workgroups (combine_kernel merges)."""
    print(f"range cache prefill which={which} D={D} L={L} S={S} causal={causal}", flush=True)
    B, Hq, Hkv, bits = 1, 8, 2, 8
    kmul, vmul = (4e4, 1.0) if which == "keys" else (1.0, 4e4)
    k, v = big_rows(B, Hkv, S, D, 1, kmul, vmul, 300 + D + L)
    cache = QuantizedKVCache(group_size=64, bits=bits)
    half = S // 2
    cache.update_and_fetch(k[:, :, :half], v[:, :, :half])  # two appends: the word is a running max
    kt, vt = cache.update_and_fetch(k[:, :, half:], v[:, :, half:])
    ek, ev = cache.range_exponents()
    assert (ek, ev) == (oracle_range(kt, bits), oracle_range(vt, bits))
    assert (ek > 0) == (which == "keys") and (ev > 0) == (which == "values")
    assert not cache.fits_fp16_operands()
    q = seeded_normal((B, Hq, L, D), 302 + L, torch.bfloat16, DEV)
    scale = 1.0 / math.sqrt(D)
    out = A.blocked_quantized_sdpa(q, kt, vt, scale, "causal" if causal else None, 64, bits)
    torch.cuda.synchronize()
    check_against_exact(out, q, kt, vt, scale, bits, ek, f"cache prefill {which} D={D}", causal=causal)
    # the same views through the one-shot kernel call, and with the word computed on the host side
    out2 = kernels.attention(q, kt, vt, scale, causal=causal, bits=bits, kernel="prefill")
    torch.cuda.synchronize()
    assert torch.equal(out, out2)


@pytest.mark.parametrize("which", ["keys", "values"])
def test_one_shot_call_on_foreign_triples_is_finite(which):
    """Triples that carry no registered word: the one-shot call computes the word from their
    scales and biases on the device."""
    print(f"range foreign triples which={which}", flush=True)
    B, Hq, Hkv, L, S, D, bits = 1, 8, 2, 64, 700, 128, 4
    kmul, vmul = (4e4, 1.0) if which == "keys" else (1.0, 4e4)
    kt, vt = big_cache(B, Hkv, S, D, bits, 1, kmul, vmul, 330)
    assert kernels.range_word(kt[0]) is None
    assert int(kernels.range_exponent(kt, bits)) == oracle_range(kt, bits)
    q = seeded_normal((B, Hq, L, D), 332, torch.bfloat16, DEV)
    scale = 1.0 / math.sqrt(D)
    out = kernels.attention(q, kt, vt, scale, causal=True, bits=bits, kernel="prefill")
    torch.cuda.synchronize()
    check_against_exact(out, q, kt, vt, scale, bits, oracle_range(kt, bits), f"foreign {which}", causal=True)


@pytest.mark.parametrize("which", ["keys", "values"])
@pytest.mark.parametrize("D", [128, 256])
def test_raw_prefill_without_a_range_word_poisons(which, D):
    """A prepared call over triples with no range word passes a null word: the row blocks that read
    an out-of-range group return NaN, the other KV head stays exact."""
    print(f"range raw prefill which={which} D={D}", flush=True)
    B, Hq, Hkv, L, S, bits = 1, 8, 2, 64, 700, 8
    kmul, vmul = (4e4, 1.0) if which == "keys" else (1.0, 4e4)
    kt, vt = big_cache(B, Hkv, S, D, bits, 1, kmul, vmul, 300)
    assert float((kt[2] if which == "keys" else vt[2])[:, 1].float().abs().max()) > 65504
    # the host-side check flags exactly the cache that the unscaled operands cannot hold
    assert not kernels.fits_fp16_operands(kt if which == "keys" else vt, bits)
    assert kernels.fits_fp16_operands(vt if which == "keys" else kt, bits)
    q = seeded_normal((B, Hq, L, D), 302, torch.bfloat16, DEV)
    scale = 1.0 / math.sqrt(D)
    out = kernels.prepare_attention(q, kt, vt, scale, causal=True, bits=bits, kernel="prefill")()
    torch.cuda.synchronize()
    o = out.cpu().float()
    assert torch.isnan(o[:, 4:]).all()
    ref = exact_reference(q[:, :4], tuple(t[:, :1] for t in kt), tuple(t[:, :1] for t in vt), scale, bits=bits,
                          causal=True)
    assert_close(out[:, :4], ref, "in-range head")


def test_paged_prefill_through_the_pool_is_finite():
    """Paged pools keep a range word too: the paged append raises it, the paged prefill reads it."""
    print("range paged prefill", flush=True)
    Hq, Hkv, D, S, L, bits = 8, 2, 128, 700, 64, 8
    cache = PagedRadixKVCache(1, Hkv, D, max_blocks=32, bits=bits, dtype=torch.bfloat16)
    k, v = big_rows(1, Hkv, S, D, 1, 1.0, 4e4, 340)
    m = cache.match_and_allocate(list(range(S)), 16)
    t = cache.tables([m.block_table])
    cache.append(0, k, v, t)
    kp, vp = cache.k_cache(0), cache.v_cache(0)
    assert int(kernels.range_word(vp[0])) > 0 and int(kernels.range_word(kp[0])) == 0
    q = seeded_normal((1, Hq, L, D), 342, torch.bfloat16, DEV)
    sl = torch.tensor([S], dtype=torch.int32, device=DEV)
    scale = 1.0 / math.sqrt(D)
    out = kernels.paged_attention(q, kp, vp, t, sl, scale, causal=True, bits=bits, max_len=S, kernel="prefill")
    torch.cuda.synchronize()
    kt, vt = cache.gather(0, m.block_table, S)
    check_against_exact(out, q, kt, vt, scale, bits, 0, "paged prefill values", causal=True)


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


def test_in_range_caches_are_unchanged():
    """A cache inside the range keeps E = 0: the prefill output is bit-identical with and without
    its word (the word changes nothing unless values leave the range)."""
    print("range in-range unchanged", flush=True)
    B, Hq, Hkv, L, S, D, bits = 1, 16, 4, 96, 900, 128, 8
    k = seeded_normal((B, Hkv, S, D), 350, torch.bfloat16, DEV)
    v = seeded_normal((B, Hkv, S, D), 351, torch.bfloat16, DEV)
    cache = QuantizedKVCache(group_size=64, bits=bits)
    kt, vt = cache.update_and_fetch(k, v)
    assert cache.range_exponents() == (0, 0)
    q = seeded_normal((B, Hq, L, D), 352, torch.bfloat16, DEV)
    a = A.blocked_quantized_sdpa(q, kt, vt, 0.09, "causal", 64, bits)
    raw = tuple(x.clone() for x in kt), tuple(x.clone() for x in vt)
    b = kernels.prepare_attention(q, raw[0], raw[1], 0.09, causal=True, bits=bits, kernel="prefill")()
    torch.cuda.synchronize()
    assert torch.equal(a, b)
