"""Pins oracle.attention.original_sdpa, the restated L == 1 / short-S hand-off of
m5engine/attention.py:42-45 (mlx-lm 0.31.3's quantized_scaled_dot_product_attention), and the
dispatch of reference_sdpa into it.

With fp32 queries, scales and biases every cast to T is exact to fp32 rounding, so the function
must equal the exact fp64 attention over the dequantized cache (to 1e-5) for every mask kind the
reference passes: None, the string "causal", a boolean [L, S] mask, a boolean per-sequence mask of
rank 4 (the GQA expand_dims path) and an additive float mask. The additive path is pinned by an
identity, not by restating it: adding log(c) to a key's score is the same as repeating that key
c times. One fp16 case is checked against a scalar brute force that applies the rounding points
of the hand-off (q*scale -> T, dequantized weights in T, scores -> T, softmax in fp32 -> T,
P.V -> T) one element at a time.
"""

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import quantize as Q


def _fp32_triple(x, bits=8, G=64):
    c, s, b = Q.quantize_values(x, G, bits)
    return (torch.from_numpy(Q.pack(c, bits).astype(np.int64)), torch.from_numpy(s), torch.from_numpy(b))


def _dequant32(x, bits=8, G=64):
    c, s, b = Q.quantize_values(x, G, bits)
    sh = x.shape
    return (c.reshape(*sh[:-1], sh[-1] // G, G) * s[..., None] + b[..., None]).reshape(sh).astype(np.float64)


def _inputs(seed, B, hq, hk, L, S, D=64):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, hq, L, D)).astype(np.float32)
    k = rng.standard_normal((B, hk, S, D)).astype(np.float32)
    v = rng.standard_normal((B, hk, S, D)).astype(np.float32)
    return q, k, v


@pytest.mark.parametrize("hq,hk", [(4, 4), (8, 2)])
@pytest.mark.parametrize("L,S", [(1, 37), (5, 96), (7, 7)])
@pytest.mark.parametrize("mask_kind", [None, "causal", "bool", "bool4", "additive_causal"])
def test_fp32_equals_exact(hq, hk, L, S, mask_kind):
    B = 2
    q, k, v = _inputs(11 + L + S, B, hq, hk, L, S)
    kt, vt = _fp32_triple(k), _fp32_triple(v)
    causal_m = torch.arange(S - L, S)[:, None] >= torch.arange(S)[None]
    seq_lens = None
    causal = mask_kind in ("causal", "bool", "additive_causal")
    if mask_kind == "bool":
        mask = causal_m
    elif mask_kind == "bool4":
        # a right-padded batch as a rank-4 boolean mask [B, 1, L, S]: sequence b has S_b keys
        seq_lens = [S, S - 3]
        mask = torch.zeros(B, 1, L, S, dtype=torch.bool)
        for b in range(B):
            mask[b, 0, :, :seq_lens[b]] = True
    elif mask_kind == "additive_causal":
        mask = torch.where(causal_m, torch.zeros(()), torch.full((), -1e9))
    else:
        mask = mask_kind
    got = A.original_sdpa(torch.from_numpy(q), kt, vt, 0.125, mask, 64, 8).numpy()
    ref = A.exact_attention(q, _dequant32(k), _dequant32(v), 0.125, causal=causal,
                            seq_lens=seq_lens)
    assert got.shape == (B, hq, L, 64)
    assert np.abs(got - ref).max() < 1e-5


@pytest.mark.parametrize("hq,hk,L", [(4, 4, 1), (8, 2, 3)])
def test_additive_mask_is_key_multiplicity(hq, hk, L):
    """softmax(s + log c) weights key j by c_j: the same as a cache where key j appears c_j
    times. Pins the additive branch (scores + mask, then softmax) by that identity."""
    S = 40
    q, k, v = _inputs(7, 1, hq, hk, L, S)
    counts = np.random.default_rng(8).integers(1, 4, size=S)
    idx = np.repeat(np.arange(S), counts)
    add = torch.from_numpy(np.log(counts).astype(np.float32))[None, :].expand(L, S).contiguous()
    got = A.original_sdpa(torch.from_numpy(q), _fp32_triple(k), _fp32_triple(v), 0.2, add, 64, 8).numpy()
    ref = A.exact_attention(q, _dequant32(k)[:, :, idx], _dequant32(v)[:, :, idx], 0.2)
    assert np.abs(got - ref).max() < 1e-5
    # a per-row constant shift changes nothing (softmax invariance)
    shift = add + torch.arange(L, dtype=torch.float32)[:, None] * 3.0
    got2 = A.original_sdpa(torch.from_numpy(q), _fp32_triple(k), _fp32_triple(v), 0.2, shift, 64, 8).numpy()
    assert np.abs(got2 - got).max() < 1e-5


def test_reference_sdpa_hands_off_to_original():
    """m5engine/attention.py:42-45: L == 1 or S <= block goes to the original SDPA unchanged."""
    q, k, v = _inputs(3, 1, 8, 2, 1, 300)
    kt, vt = _fp32_triple(k), _fp32_triple(v)
    qq = torch.from_numpy(q).half()
    kh = (kt[0], kt[1].half(), kt[2].half())
    vh = (vt[0], vt[1].half(), vt[2].half())
    # L == 1 with a block far smaller than S still takes the hand-off
    a = A.reference_sdpa(qq, kh, vh, 0.1, None, 64, 8, score_budget_bytes=1, min_block=16)
    b = A.original_sdpa(qq, kh, vh, 0.1, None, 64, 8)
    assert torch.equal(a, b)
    # short S (S <= block) with L > 1
    q2, k2, v2 = _inputs(4, 1, 4, 4, 6, 200)
    kt2, vt2 = _fp32_triple(k2), _fp32_triple(v2)
    q2h = torch.from_numpy(q2).half()
    k2h = (kt2[0], kt2[1].half(), kt2[2].half())
    v2h = (vt2[0], vt2[1].half(), vt2[2].half())
    a = A.reference_sdpa(q2h, k2h, v2h, 0.1, "causal", 64, 8)
    b = A.original_sdpa(q2h, k2h, v2h, 0.1, "causal", 64, 8)
    assert torch.equal(a, b)


def _f16(x):
    return float(np.float16(x))


def _brute_fp16(q, kc, ks, kb, vc, vs, vb, scale, L, S, causal):
    """Scalar restatement of the hand-off at T = fp16, one element at a time in numpy float16 /
    Python floats. q [Hq, L, D] fp16 values; kc/vc codes [Hkv, S, D]; ks/kb/vs/vb [Hkv, S, D/64]."""
    Hq, _, D = q.shape
    Hkv = kc.shape[0]
    rep = Hq // Hkv
    G = 64

    def w(c, s, b, h, j, d):  # dequantized weight in T: T(T(code) * scale) + bias, rounded to T
        g = d // G
        return _f16(_f16(float(c[h, j, d]) * float(s[h, j, g])) + float(b[h, j, g]))

    out = np.zeros((Hq, L, D))
    for h in range(Hq):
        kv = h // rep
        for l in range(L):
            qs = [_f16(np.float32(q[h, l, d]) * np.float32(scale)) for d in range(D)]
            sc = []
            for j in range(S):
                acc = np.float32(0.0)
                for d in range(D):
                    acc = np.float32(acc + np.float32(qs[d]) * np.float32(w(kc, ks, kb, kv, j, d)))
                s = _f16(acc)
                if causal and j > S - L + l:
                    s = float(np.finfo(np.float16).min)
                sc.append(s)
            mx = max(sc)
            e = [math.exp(s - mx) for s in sc]
            z = sum(e)
            p = [_f16(x / z) for x in e]
            for d in range(D):
                acc = 0.0
                for j in range(S):
                    acc += p[j] * w(vc, vs, vb, kv, j, d)
                out[h, l, d] = _f16(acc)
    return out


@pytest.mark.parametrize("L,causal", [(1, False), (3, True)])
def test_fp16_matches_scalar_brute_force(L, causal):
    rng = np.random.default_rng(21)
    Hq, Hkv, S, D = 4, 2, 9, 64
    q16 = rng.standard_normal((1, Hq, L, D)).astype(np.float16)
    k = rng.standard_normal((1, Hkv, S, D)).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((1, Hkv, S, D)).astype(np.float16).astype(np.float32)
    kc_, ks_, kb_ = Q.quantize_values(k, 64, 8)
    vc_, vs_, vb_ = Q.quantize_values(v, 64, 8)
    ks16, kb16, vs16, vb16 = (x.astype(np.float16) for x in (ks_, kb_, vs_, vb_))
    kt = (torch.from_numpy(Q.pack(kc_, 8).astype(np.int64)), torch.from_numpy(ks16), torch.from_numpy(kb16))
    vt = (torch.from_numpy(Q.pack(vc_, 8).astype(np.int64)), torch.from_numpy(vs16), torch.from_numpy(vb16))
    scale = 1.0 / math.sqrt(D)
    got = A.original_sdpa(torch.from_numpy(q16), kt, vt, scale, "causal" if causal else None, 64, 8)
    assert got.dtype == torch.float16
    ref = _brute_fp16(q16[0], kc_[0], ks16[0], kb16[0], vc_[0], vs16[0], vb16[0], scale, L, S, causal)
    g = got[0].float().numpy()
    # fp32 sums in a different order may move a rounding to T by one fp16 ulp; nothing more
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(g - ref) <= ulp + 1e-12)
    assert np.mean(g == ref) > 0.9
