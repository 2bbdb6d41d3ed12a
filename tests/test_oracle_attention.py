"""Pins the attention oracles (oracle/attention.py).

exact_attention is checked against a scalar brute force on tiny shapes and against closed forms
that a dropped term, a wrong GQA index or a transposed operand would break; reference_sdpa (the
port of m5engine/attention.py's blocked path) is checked with the reference's own
dense-equivalence cases (tests/test_core.py:23-40: D=64, S=700, L=6, forced 128-key blocks).
"""

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import quantize as Q


def brute(q, K, V, scale, causal, window, seq_lens):
    B, Hq, L, D = q.shape
    Hkv, S = K.shape[1], K.shape[2]
    rep = Hq // Hkv
    out = np.zeros((B, Hq, L, V.shape[-1]))
    for b in range(B):
        Sb = S if seq_lens is None else seq_lens[b]
        for h in range(Hq):
            for l in range(L):
                pos = Sb - L + l
                ks = [k for k in range(Sb) if (not causal or k <= pos) and (window <= 0 or k > pos - window)]
                if not ks:
                    continue
                s = [scale * sum(q[b, h, l, d] * K[b, h // rep, k, d] for d in range(D)) for k in ks]
                m = max(s)
                w = [math.exp(x - m) for x in s]
                z = sum(w)
                for d in range(V.shape[-1]):
                    out[b, h, l, d] = sum(wi * V[b, h // rep, k, d] for wi, k in zip(w, ks)) / z
    return out


@pytest.mark.parametrize("causal,window,seq_lens", [(False, 0, None), (True, 0, None), (True, 3, None),
                                                    (True, 0, [5, 7]), (False, 0, [4, 7]), (True, 2, [6, 3])])
def test_exact_matches_brute_force(causal, window, seq_lens):
    rng = np.random.default_rng(3)
    B, Hq, Hkv, L, S, D = 2, 4, 2, 3, 7, 5
    q = rng.standard_normal((B, Hq, L, D))
    K = rng.standard_normal((B, Hkv, S, D))
    V = rng.standard_normal((B, Hkv, S, D))
    got = A.exact_attention(q, K, V, 0.7, causal=causal, window=window, seq_lens=seq_lens)
    ref = brute(q, K, V, 0.7, causal, window, seq_lens)
    assert np.allclose(got, ref, atol=1e-12)


def test_closed_forms():
    rng = np.random.default_rng(4)
    D = 16
    q = rng.standard_normal((1, 2, 3, D))
    # one key: every row returns that value row
    K1 = rng.standard_normal((1, 1, 1, D))
    V1 = rng.standard_normal((1, 1, 1, D))
    assert np.allclose(A.exact_attention(q, K1, V1, 0.3), np.broadcast_to(V1[0, 0, 0], (1, 2, 3, D)))
    # identical keys: the mean of the values
    K = np.broadcast_to(rng.standard_normal(D), (1, 1, 9, D)).copy()
    V = rng.standard_normal((1, 1, 9, D))
    assert np.allclose(A.exact_attention(q, K, V, 0.3), np.broadcast_to(V[0, 0].mean(0), (1, 2, 3, D)))
    # a dominant logit selects its value row
    K = rng.standard_normal((1, 1, 9, D)) * 0.01
    K[0, 0, 4] = q[0, 0, 0] * 50.0
    out = A.exact_attention(q[:, :1, :1], K, V, 1.0)
    assert np.allclose(out[0, 0, 0], V[0, 0, 4], atol=1e-9)
    # permuting keys and values together changes nothing (non-causal)
    K = rng.standard_normal((1, 1, 9, D))
    perm = rng.permutation(9)
    a = A.exact_attention(q, K, V, 0.2)
    b = A.exact_attention(q, K[:, :, perm], V[:, :, perm], 0.2)
    assert np.allclose(a, b, atol=1e-12)
    # GQA: head h reads KV head h // rep
    q4 = rng.standard_normal((1, 4, 1, D))
    K2 = rng.standard_normal((1, 2, 5, D))
    V2 = rng.standard_normal((1, 2, 5, D))
    out = A.exact_attention(q4, K2, V2, 0.5)
    for h in range(4):
        single = A.exact_attention(q4[:, h:h + 1], K2[:, h // 2:h // 2 + 1], V2[:, h // 2:h // 2 + 1], 0.5)
        assert np.allclose(out[:, h:h + 1], single)


def test_fully_masked_rows_are_zero():
    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, 1, 2, 4))
    K = rng.standard_normal((1, 1, 6, 4))
    V = rng.standard_normal((1, 1, 6, 4))
    out = A.exact_attention(q, K, V, 1.0, causal=True, seq_lens=[1], window=0)
    # seq of 1 key, L=2: row 0 sits at position -1 and sees nothing
    assert np.all(out[0, 0, 0] == 0) and np.allclose(out[0, 0, 1], V[0, 0, 0])


@pytest.mark.parametrize("causal", [False, True])
def test_empty_sequence_is_zero(causal):
    # a batch row with no keys (seq_lens 0) returns 0 in every row; the other row is the plain
    # softmax average over its keys (a single query against all keys, checked by hand)
    rng = np.random.default_rng(6)
    q = rng.standard_normal((2, 1, 1, 4))
    K = rng.standard_normal((2, 1, 5, 4))
    V = rng.standard_normal((2, 1, 5, 4))
    out = A.exact_attention(q, K, V, 0.5, causal=causal, seq_lens=[5, 0])
    assert np.all(out[1] == 0)
    s = 0.5 * K[0, 0] @ q[0, 0, 0]
    w = np.exp(s - s.max())
    assert np.allclose(out[0, 0, 0], (w / w.sum()) @ V[0, 0])


def _fp32_triple(x, bits=8, G=64):
    c, s, b = Q.quantize_values(x, G, bits)
    return (torch.from_numpy(Q.pack(c, bits).astype(np.int64)).to(torch.int64),
            torch.from_numpy(s), torch.from_numpy(b))


@pytest.mark.parametrize("hq,hk", [(4, 4), (8, 2)])
@pytest.mark.parametrize("mask_kind", ["causal", "bool", None])
def test_reference_dense_equivalence(hq, hk, mask_kind):
    """tests/test_core.py:23-40 restated on the port: blocked (forced 128-key blocks, budget 1)
    equals dense softmax over the dequantized cache to 1e-4, in fp32."""
    rng = np.random.default_rng(0)
    L, S, D = 6, 700, 64
    q = rng.standard_normal((1, hq, L, D)).astype(np.float32)
    k = rng.standard_normal((1, hk, S, D)).astype(np.float32)
    v = rng.standard_normal((1, hk, S, D)).astype(np.float32)
    kt, vt = _fp32_triple(k), _fp32_triple(v)
    causal = torch.arange(S - L, S)[:, None] >= torch.arange(S)[None]
    mask = {"causal": "causal", "bool": causal, None: None}[mask_kind]
    out = A.reference_sdpa(torch.from_numpy(q), kt, vt, 0.125, mask, 64, 8, score_budget_bytes=1, min_block=128)
    c, s, b = Q.quantize_values(k, 64, 8)
    kdq = (c.reshape(1, hk, S, 1, 64) * s[..., None] + b[..., None]).reshape(1, hk, S, D)
    c, s, b = Q.quantize_values(v, 64, 8)
    vdq = (c.reshape(1, hk, S, 1, 64) * s[..., None] + b[..., None]).reshape(1, hk, S, D)
    ref = A.exact_attention(q, kdq, vdq, 0.125, causal=mask_kind is not None)
    assert np.abs(out.numpy() - ref).max() < 1e-4


def test_block_rule():
    # m5engine/attention.py:40-41
    assert A.block_size(1, 32, 512) == 512 * 1024**2 // (32 * 512 * 12)
    assert A.block_size(1, 64, 1) == 512 * 1024**2 // (64 * 12)
    assert A.block_size(1, 4, 6, score_budget_bytes=1, min_block=128) == 128


def test_error_stats():
    ref = np.array([3.0, 4.0])
    st = A.error_stats(ref + np.array([0.0, 0.5]), ref)
    assert st["max_abs"] == 0.5 and abs(st["rel_l2"] - 0.1) < 1e-12
